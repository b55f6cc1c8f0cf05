"""One measurement row per (impl, binning, shape, mode): the reference's
benchmark harness schema, for the implementations of this package.

Mirrors ``src/ace_bench/measure.py`` (``Row`` :27-81, ``compute_reference``
:142-186, ``_check_output`` :189-212, ``measure_case`` :280-360),
``src/ace_bench/calculator.py:23-44`` (ideal bytes and floors) and
``src/ace_bench/timing.py:48-77`` (CUDA events, a cache flush before each
rep so the rep starts with a cold cache: the reference writes 256 MiB, here
1 GiB is read, more than MI355X's 256 MB last-level cache), so a row from
this package can be put beside a row of the reference's harness:

- timing: p50 / p20 / p80 / mean / std of ``reps`` event-timed calls;
- bytes and floors: ideal bytes (fwd: x + target; fwd_bwd: 2 (x + target) +
  x), the HBM floor at MI355X's 8 TB/s, a launch floor of 5 us per kernel;
- cost: kernels and aten ops per call (``torch.profiler``), bytes the autograd
  node saves beyond its inputs, the call's peak allocation, what is still
  allocated afterwards;
- accuracy (untimed): loss and gradient against a trusted implementation on
  the same input (``|L - L_ref| / |L_ref|``, ``max|g - g_ref| / max|g_ref|``,
  ``||g - g_ref|| / ||g_ref||``) and against a float64 truth;
- HBM traffic (opt-in, ``counters=True``): bytes the library's kernels read
  from and write to HBM per call, from rocprofv3's FETCH_SIZE / WRITE_SIZE
  counters calibrated by a copy of known size (``ace_kernels.counters``), and
  their ratio to the ideal bytes.

Which implementation is trusted is the caller's choice: ``compute_reference``
calls whatever the registry holds under ``ref_impl`` / ``truth_impl`` (this
package registers only its HIP implementations; the tests register the CPU
restatement of the reference as ``"reference"`` and its float64 formula as
``"v2_recompute"``).
"""

from __future__ import annotations

import gc
import statistics
import traceback
import warnings
from dataclasses import dataclass
from typing import Callable, List, Literal, Optional, Tuple

import torch
from pydantic import BaseModel

from ace_kernels.config import ACEConfig
from ace_kernels.registry import ace_loss, get_impl

Mode = Literal["fwd", "fwd_bwd"]
Status = Literal["ok", "oom", "error", "unsupported", "capture_failed"]

PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E
LAUNCH_US = 5.0  # per-kernel launch floor (calculator.py:20-21)
# cold-cache flush: the reference writes 256 MiB (timing.py:15), sized for its
# GPU's cache; MI355X has a 256 MB last-level cache, so here 1 GiB is read
# (reads leave no dirty lines for the timed call to write back)
FLUSH_BYTES = 1 << 30


class Row(BaseModel):
    """One benchmark result (field names and meaning of measure.py:27-81).
    Byte and time fields are None when not measured."""

    impl: str
    binning: str
    mode: str
    cuda_graph: bool
    dtype: str = "float32"
    shape: str
    batch: int
    channels: int
    spatial: str
    voxels: int
    status: Status
    error: Optional[str] = None
    p50_ms: Optional[float] = None
    p20_ms: Optional[float] = None
    p80_ms: Optional[float] = None
    mean_ms: Optional[float] = None
    std_ms: Optional[float] = None
    reps: Optional[int] = None
    input_bytes: int
    target_bytes: int
    ideal_bytes: int
    effective_gbps: Optional[float] = None
    pct_peak_bw: Optional[float] = None
    bw_floor_ms: Optional[float] = None
    launch_floor_ms: Optional[float] = None
    kernels_per_call: Optional[int] = None
    aten_ops_per_call: Optional[int] = None
    saved_extra_bytes: Optional[int] = None
    peak_extra_bytes: Optional[int] = None
    allocated_after_bytes: Optional[int] = None
    checked_against: Optional[str] = None
    loss_rel_err: Optional[float] = None
    grad_rel_err: Optional[float] = None
    loss_err_truth: Optional[float] = None
    grad_err_truth: Optional[float] = None
    ref_loss_err_truth: Optional[float] = None
    ref_grad_err_truth: Optional[float] = None
    grad_l2_err: Optional[float] = None
    grad_l2_err_truth: Optional[float] = None
    ref_grad_l2_err_truth: Optional[float] = None
    # rocprofv3 counters (ace_kernels.counters), per call, library kernels only
    hbm_read_bytes: Optional[int] = None
    hbm_write_bytes: Optional[int] = None
    hbm_bytes_per_ideal: Optional[float] = None
    counted_kernels_per_call: Optional[int] = None


# ---------------------------------------------------------------- inputs


@dataclass(frozen=True)
class ShapeSpec:
    """A benchmark shape (the reference's ``ace_bench.config.ShapeSpec``)."""

    name: str
    batch: int
    channels: int
    spatial: Tuple[int, ...]
    logit_scale: float = 2.0
    target_bias: float = 0.0

    @property
    def voxels(self) -> int:
        n = 1
        for s in self.spatial:
            n *= s
        return n


def make_inputs(shape: ShapeSpec, config: ACEConfig, device: str,
                seed: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """Seeded logits ~ N(0, logit_scale^2) and uniform class labels, the
    labelled logit raised by ``target_bias`` (``src/ace_kernels/cases.py:
    52-93``, kind "logits"): index targets [B, 1, ...] for C > 1, a random
    binary mask for C == 1."""
    gen = torch.Generator().manual_seed(seed)
    full = (shape.batch, shape.channels, *shape.spatial)
    x = torch.randn(full, generator=gen) * shape.logit_scale
    labels = torch.randint(0, shape.channels, (shape.batch, 1, *shape.spatial), generator=gen)
    if shape.channels == 1:
        target = torch.randint(0, 2, labels.shape, generator=gen).float()
    elif config.to_onehot_y:
        target = labels
    else:
        target = torch.zeros(full).scatter_(1, labels, 1.0)
    if shape.target_bias and shape.channels > 1:
        x.scatter_add_(1, labels, torch.full(labels.shape, shape.target_bias, dtype=x.dtype))
    return x.to(device), target.to(device)


# ---------------------------------------------------------------- bytes and floors


def ideal_bytes(input_bytes: int, target_bytes: int, mode: Mode) -> int:
    return input_bytes + target_bytes if mode == "fwd" else 2 * (input_bytes + target_bytes) + input_bytes


def bandwidth_floor_ms(nbytes: int, peak_gbps: float = PEAK_HBM_GBPS) -> float:
    return nbytes / (peak_gbps * 1e9) * 1e3


def launch_floor_ms(kernels: int, launch_us: float = LAUNCH_US) -> float:
    return kernels * launch_us / 1e3


def effective_gbps(nbytes: int, ms: float) -> float:
    return nbytes / (ms / 1e3) / 1e9


# ---------------------------------------------------------------- timing


@dataclass
class TimingStats:
    p50_ms: float
    p20_ms: float
    p80_ms: float
    mean_ms: float
    std_ms: float
    min_ms: float
    reps: int


def _quantile(sorted_ms: List[float], q: float) -> float:
    return sorted_ms[min(len(sorted_ms) - 1, max(0, round(q * (len(sorted_ms) - 1))))]


def summarize(ms: List[float]) -> TimingStats:
    s = sorted(ms)
    return TimingStats(_quantile(s, 0.5), _quantile(s, 0.2), _quantile(s, 0.8), statistics.fmean(s),
                       statistics.stdev(s) if len(s) > 1 else 0.0, s[0], len(s))


def measure(fn: Callable[[], object], warmup: int = 5, reps: int = 20, flush: bool = True) -> TimingStats:
    """Event-timed calls of ``fn`` on the current stream, each after a read of
    FLUSH_BYTES (the reference's cold-cache method, sized for MI355X)."""
    for _ in range(warmup):
        fn()
    buf = torch.zeros(FLUSH_BYTES // 4, dtype=torch.float32, device="cuda")
    sink = torch.empty((), dtype=torch.float32, device="cuda")
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    torch.cuda.synchronize()
    for s, e in zip(starts, ends):
        if flush:
            torch.sum(buf, dim=0, out=sink)
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    del buf
    return summarize([s.elapsed_time(e) for s, e in zip(starts, ends)])


# ---------------------------------------------------------------- accuracy


@dataclass
class Reference:
    """Loss and input gradient of a trusted implementation (CPU tensors);
    ``truth_*``: a float64 evaluation on the same input values."""

    impl: str
    loss: torch.Tensor
    grad: torch.Tensor
    truth_loss: Optional[torch.Tensor] = None
    truth_grad: Optional[torch.Tensor] = None
    ref_loss_err_truth: Optional[float] = None
    ref_grad_err_truth: Optional[float] = None
    ref_grad_l2_err_truth: Optional[float] = None
    # rocprofv3 counters (ace_kernels.counters), per call, library kernels only
    hbm_read_bytes: Optional[int] = None
    hbm_write_bytes: Optional[int] = None
    hbm_bytes_per_ideal: Optional[float] = None
    counted_kernels_per_call: Optional[int] = None


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """max |a - b| / max |b| (b trusted)."""
    diff = (a.double() - b.double()).abs().max()
    return float(diff / b.double().abs().max().clamp_min(1e-12))


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    """||a - b|| / ||b|| (b trusted)."""
    diff = torch.linalg.vector_norm(a.double() - b.double())
    return float(diff / torch.linalg.vector_norm(b.double()).clamp_min(1e-30))


def loss_and_grad(impl: str, x: torch.Tensor, y: torch.Tensor,
                  config: ACEConfig) -> Tuple[torch.Tensor, torch.Tensor]:
    leaf = x.detach().requires_grad_(True)
    loss = ace_loss(leaf, y, config, impl=impl)
    (grad,) = torch.autograd.grad(loss.sum(), leaf)
    return loss.detach().float().cpu(), grad.float().cpu()


def compute_reference(shape: ShapeSpec, config: ACEConfig, device: str = "cpu", seed: int = 0,
                      dtype: torch.dtype = torch.float32, ref_impl: str = "reference",
                      truth_impl: Optional[str] = "v2_recompute") -> Reference:
    """``ref_impl`` on the benchmark input, and ``truth_impl`` in float64 on the
    same (already rounded) values (measure.py:142-186)."""
    x, y = make_inputs(shape, config, device, seed)
    x = x.to(dtype)
    loss, grad = loss_and_grad(ref_impl, x, y, config)
    ref = Reference(ref_impl, loss, grad)
    if truth_impl is not None:
        leaf = x.detach().double().requires_grad_(True)
        loss64 = ace_loss(leaf, y, config, impl=truth_impl)
        (grad64,) = torch.autograd.grad(loss64.sum(), leaf)
        ref.truth_loss, ref.truth_grad = loss64.detach().cpu(), grad64.cpu()
        ref.ref_loss_err_truth = rel_err(ref.loss, ref.truth_loss)
        ref.ref_grad_err_truth = rel_err(ref.grad, ref.truth_grad)
        ref.ref_grad_l2_err_truth = rel_l2(ref.grad, ref.truth_grad)
    return ref


def check_output(row: Row, impl: str, x: torch.Tensor, y: torch.Tensor, config: ACEConfig,
                 ref: Reference) -> None:
    """Fill the row's error columns (measure.py:189-212)."""
    row.checked_against = ref.impl
    row.ref_loss_err_truth = ref.ref_loss_err_truth
    row.ref_grad_err_truth = ref.ref_grad_err_truth
    row.ref_grad_l2_err_truth = ref.ref_grad_l2_err_truth
    loss, grad = loss_and_grad(impl, x, y, config)
    row.loss_rel_err, row.grad_rel_err = rel_err(loss, ref.loss), rel_err(grad, ref.grad)
    row.grad_l2_err = rel_l2(grad, ref.grad)
    if ref.truth_loss is not None and ref.truth_grad is not None:
        row.loss_err_truth = rel_err(loss, ref.truth_loss)
        row.grad_err_truth = rel_err(grad, ref.truth_grad)
        row.grad_l2_err_truth = rel_l2(grad, ref.truth_grad)


# ---------------------------------------------------------------- cost


def step_fn(impl: str, x: torch.Tensor, y: torch.Tensor, config: ACEConfig,
            mode: Mode) -> Callable[[], object]:
    def fwd() -> torch.Tensor:
        return ace_loss(x, y, config, impl=impl)

    def fwd_bwd() -> torch.Tensor:
        (grad,) = torch.autograd.grad(fwd().sum(), x)
        return grad

    return fwd if mode == "fwd" else fwd_bwd


def graphed(fn: Callable[[], object]) -> Callable[[], object]:
    """Capture ``fn`` in a HIP graph (warm-up on a side stream first); the
    returned callable replays it."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        fn()
    return graph.replay


def count_ops(fn: Callable[[], object]) -> Tuple[int, int]:
    """Device kernels and aten ops of one call."""
    from torch.profiler import ProfilerActivity, profile

    with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
        fn()
        torch.cuda.synchronize()
    events = prof.events()
    kernels = sum(1 for e in events if e.device_type.name == "CUDA")
    aten = sum(1 for e in events if e.name.startswith("aten::"))
    return kernels, aten


def saved_extra_bytes(fn: Callable[[], object], exclude: List[torch.Tensor]) -> int:
    """Bytes the autograd graph of ``fn()`` saves beyond the tensors in
    ``exclude`` (storage identity), counted once per storage."""
    seen, total = set(), 0
    skip = {t.untyped_storage().data_ptr() for t in exclude}

    def pack(t: torch.Tensor):
        nonlocal total
        key = t.untyped_storage().data_ptr()
        if key not in skip and key not in seen:
            seen.add(key)
            total += t.untyped_storage().nbytes()
        return t

    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
        out = fn()
    del out
    return total


def peak_extra_bytes(fn: Callable[[], object]) -> int:
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = fn()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - before
    del out
    return peak


def release_memory() -> None:
    gc.collect()
    torch.cuda.empty_cache()


# ---------------------------------------------------------------- one row


def fill_counters(row: Row, impl: str, shape: ShapeSpec, config: ACEConfig, mode: Mode,
                  dtype: torch.dtype, seed: int, calls: int = 10) -> None:
    """The row's HBM traffic columns from two rocprofv3 counter runs of the
    same case in child processes (ace_kernels.counters)."""
    from ace_kernels import counters

    case = counters.CaseArgs(impl=impl, config=config.model_dump_json(), batch=shape.batch,
                             channels=shape.channels, spatial=tuple(shape.spatial),
                             logit_scale=shape.logit_scale, target_bias=shape.target_bias,
                             mode=mode, dtype=str(dtype).replace("torch.", ""), seed=seed,
                             calls=calls)
    tr = counters.collect(case)
    row.hbm_read_bytes = round(tr.read_bytes)
    row.hbm_write_bytes = round(tr.write_bytes)
    row.hbm_bytes_per_ideal = tr.total_bytes / row.ideal_bytes
    row.counted_kernels_per_call = tr.dispatches


def measure_case(impl: str, shape: ShapeSpec, config: ACEConfig, mode: Mode, *,
                 cuda_graph: bool = False, warmup: int = 3, reps: int = 10, seed: int = 0,
                 reference: Optional[Reference] = None, dtype: torch.dtype = torch.float32,
                 peak_gbps: float = PEAK_HBM_GBPS, counters: bool = False) -> Row:
    """measure.py:280-360 for one case on the current HIP device; with
    ``counters`` also the HBM traffic columns (not for graph rows; a counter
    failure is recorded in ``error`` and leaves the timing columns)."""
    x, y = make_inputs(shape, config, "cuda", seed)
    x = x.to(dtype).requires_grad_(True)
    in_bytes = x.numel() * x.element_size()
    tgt_bytes = y.numel() * y.element_size()
    ideal = ideal_bytes(in_bytes, tgt_bytes, mode)
    row = Row(impl=impl, binning=config.binning, mode=mode, cuda_graph=cuda_graph,
              dtype=str(dtype).replace("torch.", ""), shape=shape.name, batch=shape.batch,
              channels=shape.channels, spatial="x".join(map(str, shape.spatial)),
              voxels=shape.voxels, status="ok", input_bytes=in_bytes, target_bytes=tgt_bytes,
              ideal_bytes=ideal, bw_floor_ms=bandwidth_floor_ms(ideal, peak_gbps))
    if not get_impl(impl).supports(config.binning, "cuda"):
        row.status = "unsupported"
        return row
    fn = step_fn(impl, x, y, config, mode)
    try:
        with warnings.catch_warnings():
            warnings.simplefilter("ignore", UserWarning)
            fn()  # allocator / first-call warm-up, untimed
            if cuda_graph:
                try:
                    fn = graphed(fn)
                except Exception as exc:  # noqa: BLE001 -- recorded in the row
                    row.status = "capture_failed"
                    row.error = f"{type(exc).__name__}: {exc}"[:500]
                    return row
            else:
                leaf = x.detach().requires_grad_(True)
                row.saved_extra_bytes = saved_extra_bytes(
                    lambda: ace_loss(leaf, y, config, impl=impl), [leaf, y])
            row.kernels_per_call, row.aten_ops_per_call = count_ops(fn)
            row.launch_floor_ms = launch_floor_ms(row.kernels_per_call)
            if not cuda_graph:
                row.peak_extra_bytes = peak_extra_bytes(fn)
            st = measure(fn, warmup=warmup, reps=reps)
            row.p50_ms, row.p20_ms, row.p80_ms = st.p50_ms, st.p20_ms, st.p80_ms
            row.mean_ms, row.std_ms, row.reps = st.mean_ms, st.std_ms, st.reps
            row.effective_gbps = effective_gbps(ideal, st.p50_ms)
            row.pct_peak_bw = 100.0 * row.effective_gbps / peak_gbps
            if reference is not None and not cuda_graph:
                del fn
                check_output(row, impl, x, y, config, reference)
            if counters and not cuda_graph:
                try:
                    fill_counters(row, impl, shape, config, mode, dtype, seed)
                except Exception as exc:  # noqa: BLE001 -- recorded in the row
                    row.error = ("counters: " + "".join(
                        traceback.format_exception_only(exc)).strip())[:500]
    except torch.OutOfMemoryError as exc:
        row.status, row.error = "oom", str(exc).splitlines()[0][:500]
    except Exception as exc:  # noqa: BLE001 -- recorded in the row
        row.status = "error"
        row.error = "".join(traceback.format_exception_only(exc)).strip()[:500]
    release_memory()
    row.allocated_after_bytes = torch.cuda.memory_allocated()
    return row


def main(argv: Optional[List[str]] = None) -> int:
    """``python -m ace_kernels.measure``: rows (JSON lines) of this package's
    implementations on the reference's paper shapes, no output check."""
    import argparse
    import json

    ap = argparse.ArgumentParser(description=main.__doc__)
    ap.add_argument("--impls", default="hip_mi355x,hip_mi355x_op")
    ap.add_argument("--binnings", default="hard,soft")
    ap.add_argument("--modes", default="fwd,fwd_bwd")
    ap.add_argument("--graph", action="store_true", help="also the HIP-graph rows")
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--counters", action="store_true",
                    help="also HBM read / write bytes per call (two rocprofv3 counter runs per row)")
    args = ap.parse_args(argv)
    import ace_kernels  # noqa: F401 -- registers the implementations

    shapes = [ShapeSpec("kits23", 2, 4, (128, 128, 128)), ShapeSpec("ds2-32", 1, 4, (32, 32, 32))]
    for shape in shapes:
        for binning in args.binnings.split(","):
            cfg = ACEConfig(binning=binning, num_bins=20, to_onehot_y=True, activation="softmax")
            for impl in args.impls.split(","):
                for mode in args.modes.split(","):
                    for graph in ((False, True) if args.graph else (False,)):
                        row = measure_case(impl, shape, cfg, mode, cuda_graph=graph, reps=args.reps,
                                           counters=args.counters)
                        print(json.dumps(row.model_dump()), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
