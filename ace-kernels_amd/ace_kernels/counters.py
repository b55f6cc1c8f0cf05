"""HBM traffic of one measurement case from rocprofv3 hardware counters.

The reference's harness profiles with torch.profiler and Nsight Systems
(``src/ace_bench/profile.py:1-13``); on MI355X the bytes a kernel moves to
and from HBM come from two rocprofv3 counter runs, one counter each (a run
takes at most 4 TCC counters and FETCH_SIZE alone uses 3):

- ``FETCH_SIZE`` and ``WRITE_SIZE`` per dispatch, in KiB;
- both scaled by what they read for a plain copy of known size (256 MiB read
  and 256 MiB written) that the same run makes after the case, since
  FETCH_SIZE does not count every fetched byte one for one.

Each run is a child process, ``rocprofv3 --pmc <counter> -- python -m
ace_kernels.counters --child <case>``, that rebuilds the case from its
arguments (or takes a benchmark configuration's inputs), calls it ``calls``
times, then copies the calibration tensor ``calls`` times.  The per-call bytes are the counters of every dispatch whose
kernel name contains ``kernel_filter`` (the library's kernels by default),
summed and divided by ``calls``.
"""

from __future__ import annotations

import csv
import json
import os
import shutil
import signal
import statistics
import subprocess
import sys
import tempfile
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Dict, List, Optional, Tuple

COPY_BYTES = 256 << 20  # calibration copy: read and written once per call
COUNTERS = ("FETCH_SIZE", "WRITE_SIZE")
KERNEL_FILTER = "ace::"


@dataclass(frozen=True)
class CaseArgs:
    """Everything the child needs to rebuild a measurement case."""

    impl: str
    config: str  # ACEConfig as JSON
    batch: int
    channels: int
    spatial: Tuple[int, ...]
    logit_scale: float
    target_bias: float
    mode: str
    dtype: str  # torch dtype name, e.g. "float32"
    seed: int
    calls: int = 10
    workload: int = 0  # > 0: the inputs and config of benchmark configuration `workload`

    def to_argv(self) -> List[str]:
        return ["--child", json.dumps(asdict(self))]

    @staticmethod
    def from_json(text: str) -> "CaseArgs":
        d = json.loads(text)
        d["spatial"] = tuple(d["spatial"])
        return CaseArgs(**d)


@dataclass
class Traffic:
    """Bytes per call of the matched kernels, scaled by the copy calibration."""

    read_bytes: float
    write_bytes: float
    fetch_kib: float      # raw counter sums per call
    write_kib: float
    fetch_scale: float    # COPY_BYTES / 1024 over the copy's FETCH_SIZE
    write_scale: float
    dispatches: int       # matched dispatches per call

    @property
    def total_bytes(self) -> float:
        return self.read_bytes + self.write_bytes


def parse_counter_csv(paths: List[Path]) -> Dict[str, List[Tuple[str, float]]]:
    """counter name -> [(kernel name, value)] over the dispatches of every
    ``*counter_collection.csv`` in ``paths``, in file order."""
    out: Dict[str, List[Tuple[str, float]]] = {}
    for p in paths:
        with open(p, newline="") as fh:
            for r in csv.DictReader(fh):
                out.setdefault(r["Counter_Name"], []).append(
                    (r["Kernel_Name"], float(r["Counter_Value"])))
    return out


def copy_value(rows: List[Tuple[str, float]]) -> Optional[float]:
    """The calibration copy's counter value: the median over the copy-kernel
    dispatches within a factor of two of the largest (smaller copies of the
    case itself, if any, are left out)."""
    vals = [v for name, v in rows if "copyBuffer" in name]
    if not vals:
        return None
    big = [v for v in vals if v >= 0.5 * max(vals)]
    return statistics.median(big)


def per_call(rows: List[Tuple[str, float]], calls: int, kernel_filter: str) -> Tuple[float, int]:
    """Sum of the matched dispatches' values per call, and matched dispatches
    per call."""
    vals = [v for name, v in rows if kernel_filter in name]
    return sum(vals) / calls, len(vals) // calls


def traffic_from_rows(fetch: List[Tuple[str, float]], write: List[Tuple[str, float]], calls: int,
                      kernel_filter: str = KERNEL_FILTER) -> Traffic:
    fc, wc = copy_value(fetch), copy_value(write)
    if not fc or not wc:
        raise RuntimeError("no calibration copy among the counted dispatches")
    copy_kib = COPY_BYTES / 1024.0
    fs, ws = copy_kib / fc, copy_kib / wc
    f_kib, n = per_call(fetch, calls, kernel_filter)
    w_kib, _ = per_call(write, calls, kernel_filter)
    if n == 0:
        raise RuntimeError(f"no dispatch of a kernel matching {kernel_filter!r} was counted")
    return Traffic(read_bytes=f_kib * fs * 1024.0, write_bytes=w_kib * ws * 1024.0,
                   fetch_kib=f_kib, write_kib=w_kib, fetch_scale=fs, write_scale=ws, dispatches=n)


def rocprof() -> str:
    for cand in (os.environ.get("ROCPROFV3"), "/opt/rocm/bin/rocprofv3", shutil.which("rocprofv3")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("rocprofv3 not found (set ROCPROFV3 or install ROCm under /opt/rocm)")


def _child_env() -> Dict[str, str]:
    """The child imports this package from the same place as the parent."""
    env = dict(os.environ)
    pkg_root = str(Path(__file__).resolve().parent.parent)
    env["PYTHONPATH"] = pkg_root + (os.pathsep + env["PYTHONPATH"] if env.get("PYTHONPATH") else "")
    return env


def collect(case: CaseArgs, timeout: float = 120.0, kernel_filter: str = KERNEL_FILTER) -> Traffic:
    """Two rocprofv3 runs of the case (FETCH_SIZE, then WRITE_SIZE) -> Traffic.
    Each run is killed after ``timeout`` seconds."""
    rows: Dict[str, List[Tuple[str, float]]] = {}
    with tempfile.TemporaryDirectory(prefix="ace_counters_") as tmp:
        for counter in COUNTERS:
            out = Path(tmp) / counter
            cmd = [rocprof(), "--pmc", counter, "--output-format", "csv", "-d", str(out), "-o", "run",
                   "--", sys.executable, "-m", "ace_kernels.counters", *case.to_argv()]
            # its own process group, so that a run past the limit is killed
            # with every process it started
            proc = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                                    env=_child_env(), start_new_session=True)
            try:
                text, _ = proc.communicate(timeout=timeout)
            except subprocess.TimeoutExpired:
                os.killpg(proc.pid, signal.SIGKILL)
                proc.communicate()
                raise RuntimeError(f"rocprofv3 --pmc {counter} ran past {timeout:.0f} s") from None
            files = sorted(out.rglob("*counter_collection.csv"))
            # the profiler may exit non-zero after the child finished and its
            # results were written: the child's last line says it finished
            finished = "counted " in (text or "")
            if not files or (proc.returncode != 0 and not finished):
                raise RuntimeError(f"rocprofv3 --pmc {counter} failed (exit {proc.returncode}):\n"
                                   f"{(text or '')[-2000:]}")
            rows[counter] = parse_counter_csv(files).get(counter, [])
    return traffic_from_rows(rows["FETCH_SIZE"], rows["WRITE_SIZE"], case.calls, kernel_filter)


def _run_child(case: CaseArgs) -> int:
    import torch

    import ace_kernels  # noqa: F401 -- registers the implementations
    from ace_kernels.config import ACEConfig
    from ace_kernels.measure import ShapeSpec, make_inputs, step_fn

    if case.workload > 0:
        from ace_kernels.workloads import workload

        wl = workload(case.workload)
        cfg = wl.config
        x, y = wl.make("cuda")
        x = x.requires_grad_(True)
    else:
        cfg = ACEConfig.model_validate_json(case.config)
        shape = ShapeSpec("counted", case.batch, case.channels, case.spatial, case.logit_scale,
                          case.target_bias)
        x, y = make_inputs(shape, cfg, "cuda", case.seed)
        x = x.to(getattr(torch, case.dtype)).requires_grad_(True)
    fn = step_fn(case.impl, x, y, cfg, case.mode)  # type: ignore[arg-type]
    # no warm-up call: every call of the case is counted and divided by calls
    for _ in range(case.calls):
        fn()
    torch.cuda.synchronize()
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(case.calls):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"counted {case.calls} calls of {case.impl} {case.mode} and {case.calls} copies", flush=True)
    return 0


def main(argv: Optional[List[str]] = None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    if len(argv) != 2 or argv[0] != "--child":
        print("usage: python -m ace_kernels.counters --child '<case JSON>' (run under rocprofv3)",
              file=sys.stderr)
        return 2
    return _run_child(CaseArgs.from_json(argv[1]))


if __name__ == "__main__":
    raise SystemExit(main())
