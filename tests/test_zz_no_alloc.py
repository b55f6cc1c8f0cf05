"""ace_forward_noalloc (the allocation-free forward) against ace_forward.

The entry point has no counterpart in the reference: it is for callers that
cannot allocate device memory.  Its workspace is the library's static device
scratch, which keeps what the last call on the device left; it launches
ace_forward's kernels, so its outputs (coef, d, jac, per-class errors, loss,
float64 statistics) must equal ace_forward's bit for bit.  Each case runs
two calls in a row, the second on a smaller problem, each checked against
ace_forward on the same inputs."""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig, _lib
from ace_kernels.common import class_weight_tensor, class_weights
from ace_kernels.impls import hip_mi355x as hip
from gpu_helpers import say

pytestmark = pytest.mark.gpu


def _inputs(b, c, spatial, seed, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn((b, c, *spatial), generator=gen) * 1.5)
    y = torch.randint(0, c, (b, 1, *spatial), generator=gen)
    x[:, 1] += 1.0  # not a uniform softmax
    return x.to(dtype).cuda(), y.cuda()


def _allocator_counts(dev):
    st = torch.cuda.memory_stats(dev)
    return st["allocation.all.allocated"], st["segment.all.allocated"]


def _noalloc(pl, config: ACEConfig):
    """The outputs of one ace_forward_noalloc call, laid out as hip_forward's."""
    lib = _lib.lib()
    dev = pl.x.device
    f32 = torch.float32
    coef = torch.empty((pl.B, pl.CL, pl.K), dtype=f32, device=dev)
    d = torch.empty(hip._d_shape(pl), dtype=f32, device=dev)  # soft: d and its remainder
    jac = torch.empty((pl.B, pl.CL), dtype=f32, device=dev)
    per_class = torch.empty((pl.B, pl.CL), dtype=f32, device=dev)
    reduction = hip._REDUCTIONS[config.reduction]
    loss = torch.empty((), dtype=f32, device=dev) if reduction != _lib.RED_NONE else None
    st = torch.empty((3, pl.B, pl.CL, pl.K), dtype=torch.float64, device=dev)
    weights = class_weights(config, pl.CL)
    cw = class_weight_tensor(tuple(weights), dev) if weights is not None else None
    torch.cuda.synchronize()
    # cumulative counts of torch's allocator (frees by the garbage collector
    # during the call do not change them)
    before = _allocator_counts(dev)
    rc = lib.ace_forward_noalloc(
        pl.x.data_ptr(), pl.dtype_code, pl.target.data_ptr(), pl.target_kind,
        pl.B, pl.C, pl.N, pl.K, _lib.SOFT if pl.soft else _lib.HARD, pl.act,
        int(pl.include_bg), int(config.ignore_empty_classes), reduction, int(pl.right),
        float(config.empty_weight), hip._ptr(cw), pl.btab.data_ptr(), hip._ptr(pl.rtab),
        coef.data_ptr(), d.data_ptr(), jac.data_ptr(), per_class.data_ptr(), hip._ptr(loss),
        st.data_ptr(), hip._stream(dev),
    )
    _lib.check(rc, "ace_forward_noalloc")
    torch.cuda.synchronize()
    # nothing allocated through torch's allocator during the call
    assert _allocator_counts(dev) == before
    if loss is None:  # reduction "none": the per-class errors, as hip_forward returns them
        loss = per_class.view(pl.B, pl.CL, *([1] * pl.spatial_ndim))
    return loss, coef, d, jac, per_class, st


CASES = {
    # (config, first problem, second (smaller) problem)
    "hard-cfg2": (ACEConfig(binning="hard", to_onehot_y=True),
                  (2, 4, (128, 128, 128), torch.float32), (1, 4, (20, 24, 28), torch.float32)),
    "soft-cfg3": (ACEConfig(binning="soft", to_onehot_y=True),
                  (2, 4, (128, 128, 128), torch.float32), (2, 4, (16, 16, 16), torch.float32)),
    "soft-cfg5": (ACEConfig(binning="soft", num_bins=50, to_onehot_y=True, include_background=False),
                  (32, 4, (512, 512), torch.bfloat16), (3, 4, (40, 36), torch.bfloat16)),
    "hard-c16": (ACEConfig(binning="hard", to_onehot_y=True, reduction="none"),
                 (1, 16, (64, 64, 64), torch.float32), (1, 16, (12, 12, 12), torch.float32)),
    "hard-generic": (ACEConfig(binning="hard", to_onehot_y=False, activation="sigmoid"),
                     (2, 3, (48, 48, 48), torch.float32), (1, 3, (10, 10, 10), torch.float32)),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_noalloc_matches_forward_on_two_calls(name: str) -> None:
    config, first, second = CASES[name]
    for i, (b, c, spatial, dtype) in enumerate((first, second)):
        x, y = _inputs(b, c, spatial, 40 + i, dtype)
        if not config.to_onehot_y:
            y = torch.nn.functional.one_hot(y[:, 0], c).movedim(-1, 1).float()
        pl = hip.make_plan(x, y, config)
        say(f"noalloc {name} call {i}: B={b} C={c} {spatial} {dtype}")
        want = hip.hip_forward(pl, config, stats=True, shared=False)
        got = _noalloc(pl, config)
        for what, g, w in zip(("loss", "coef", "d", "jac", "per_class", "stats"), got, want):
            if w is None:
                assert g is None, what
                continue
            assert torch.equal(g, w) or (torch.isnan(w).any() and torch.equal(g.isnan(), w.isnan())
                                         and torch.equal(g.nan_to_num(), w.nan_to_num())), \
                f"{name} call {i}: {what}"


def _noalloc_call(pl, config, outs, stream):
    """One ace_forward_noalloc call into preallocated outputs (no checks, no
    synchronisation: it may be captured)."""
    coef, d, jac, per_class, loss, st = outs
    weights = class_weights(config, pl.CL)
    cw = class_weight_tensor(tuple(weights), pl.x.device) if weights is not None else None
    return _lib.lib().ace_forward_noalloc(
        pl.x.data_ptr(), pl.dtype_code, pl.target.data_ptr(), pl.target_kind,
        pl.B, pl.C, pl.N, pl.K, _lib.SOFT if pl.soft else _lib.HARD, pl.act,
        int(pl.include_bg), int(config.ignore_empty_classes), hip._REDUCTIONS[config.reduction],
        int(pl.right), float(config.empty_weight), hip._ptr(cw), pl.btab.data_ptr(), hip._ptr(pl.rtab),
        coef.data_ptr(), d.data_ptr(), jac.data_ptr(), per_class.data_ptr(), hip._ptr(loss),
        st.data_ptr(), stream)


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_noalloc_replays_under_graph_capture(binning: str) -> None:
    """The main use of the entry point: captured into a HIP graph after one
    warm call, each replay (with eager work and synchronisations between the
    replays) equals ace_forward bit for bit, and a warm eager call leaves the
    device's free memory unchanged."""
    config = ACEConfig(binning=binning, to_onehot_y=True)
    x, y = _inputs(2, 4, (40, 40, 40), 61)
    pl = hip.make_plan(x, y, config)
    want = hip.hip_forward(pl, config, stats=True, shared=False)
    dev = x.device
    outs = (torch.empty((pl.B, pl.CL, pl.K), device=dev), torch.empty(hip._d_shape(pl), device=dev),
            torch.empty((pl.B, pl.CL), device=dev), torch.empty((pl.B, pl.CL), device=dev),
            torch.empty((), device=dev), torch.empty((3, pl.B, pl.CL, pl.K), dtype=torch.float64, device=dev))
    say(f"noalloc graph {binning}: warm call")
    _lib.check(_noalloc_call(pl, config, outs, hip._stream(dev)), "ace_forward_noalloc")
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info(dev)[0]
    _lib.check(_noalloc_call(pl, config, outs, hip._stream(dev)), "ace_forward_noalloc")
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(dev)[0] == free_before
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    say(f"noalloc graph {binning}: capture")
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = _noalloc_call(pl, config, outs, hip._stream(dev))
    torch.cuda.synchronize()
    _lib.check(rc, "ace_forward_noalloc (captured)")
    for r in range(3):
        for o in outs:
            o.fill_(7.0)
        say(f"noalloc graph {binning}: replay {r}")
        graph.replay()
        torch.cuda.synchronize()
        hip.hip_forward(pl, config, stats=True, shared=False)  # eager work between replays
        torch.cuda.synchronize()
        got = (outs[4], outs[0], outs[1], outs[2], outs[3], outs[5])
        for what, g, w in zip(("loss", "coef", "d", "jac", "per_class", "stats"), got, want):
            assert torch.equal(g, w), f"replay {r}: {what}"


def test_noalloc_rejects_oversize_on_the_device() -> None:
    """A problem beyond the scratch returns ACE_ESCRATCH and launches nothing."""
    config = ACEConfig(binning="soft", num_bins=50, to_onehot_y=True)
    x, y = _inputs(200, 4, (8, 8), 7)
    pl = hip.make_plan(x, y, config)
    lib = _lib.lib()
    assert lib.ace_workspace_bytes(200, 4, 64, 50, _lib.SOFT, _lib.F32, 1, 0) > _lib.NOALLOC_SCRATCH_BYTES
    out = torch.full((200 * 4 * 50,), 3.0, device="cuda")
    say("noalloc oversize")
    rc = lib.ace_forward_noalloc(
        pl.x.data_ptr(), pl.dtype_code, pl.target.data_ptr(), pl.target_kind, 200, 4, 64, 50,
        _lib.SOFT, pl.act, 1, 1, _lib.RED_MEAN, 0, 0.01, None, pl.btab.data_ptr(),
        pl.rtab.data_ptr(), out.data_ptr(), out.data_ptr(), out.data_ptr(), out.data_ptr(),
        out.data_ptr(), None, hip._stream(x.device))
    assert rc == _lib.ESCRATCH
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())
