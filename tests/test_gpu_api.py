"""The HIP path behind the other entry points: drop-in modules, the
torch.library custom ops, torch.compile, HIP graphs and host synchronisation
(upstream tests/test_module.py, tests/test_triton.py:474-495 and
tests/test_sync.py:27-97 check the same properties of the reference's impls)."""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig, ace_loss
from ace_kernels.module import HardL1ACELoss, SoftL1ACELoss
from gpu_helpers import run, say

pytestmark = pytest.mark.gpu


def _inputs(seed: int = 0, shape=(2, 4, 16, 12, 10)):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=gen) * 2.0
    y = torch.randint(0, shape[1], (shape[0], 1, *shape[2:]), generator=gen)
    return x.cuda(), y.cuda()


@pytest.mark.parametrize("cls", [HardL1ACELoss, SoftL1ACELoss])
def test_module_matches_ace_loss(cls) -> None:
    x, y = _inputs(1)
    m = cls(num_bins=20, to_onehot_y=True, softmax=True)
    say(f"module {cls.__name__}")
    assert m.resolve_impl(x.device) == "hip_mi355x"
    loss_m, grad_m = run_module(m, x, y)
    loss_r, grad_r = run("hip_mi355x", x, y, m.config)
    assert torch.equal(loss_m, loss_r) and torch.equal(grad_m, grad_r)


def run_module(m, x, y):
    leaf = x.detach().clone().requires_grad_(True)
    loss = m(leaf, y)
    (g,) = torch.autograd.grad(loss.sum(), leaf)
    return loss.detach(), g


@pytest.mark.parametrize("reduction", ["mean", "none"])
@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_custom_op_matches_autograd_function(binning, reduction) -> None:
    x, y = _inputs(2)
    cfg = ACEConfig(binning=binning, to_onehot_y=True, reduction=reduction)
    say(f"custom op {binning} {reduction}")
    upstream = torch.rand((2, 4, 1, 1, 1)) if reduction == "none" else None
    a = run("hip_mi355x", x, y, cfg, upstream)
    b = run("hip_mi355x_op", x, y, cfg, upstream)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_opcheck() -> None:
    from ace_kernels.impls.hip_mi355x import _dump

    x, y = _inputs(3, (1, 3, 8, 8, 4))
    say("opcheck hip_forward")
    for binning in ("hard", "soft"):
        cfg = _dump(ACEConfig(binning=binning, to_onehot_y=True))
        torch.library.opcheck(torch.ops.ace_kernels.hip_forward, (x.requires_grad_(True), y, cfg),
                              test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_torch_compile_fullgraph(binning) -> None:
    """A small network plus the loss compiles as one graph (fullgraph=True
    raises on any graph break) and matches eager execution."""
    torch._dynamo.reset()
    x, y = _inputs(4, (2, 3, 8, 8, 8))
    conv = torch.nn.Conv3d(3, 4, 3, padding=1).cuda()
    loss_fn = (HardL1ACELoss if binning == "hard" else SoftL1ACELoss)(
        to_onehot_y=True, softmax=True, impl="hip_mi355x_op")

    def step(inp):
        return loss_fn(conv(inp), y)

    compiled = torch.compile(step, fullgraph=True, backend="aot_eager")
    say(f"torch.compile {binning}")
    xe = x.detach().clone().requires_grad_(True)
    le = step(xe)
    (ge,) = torch.autograd.grad(le, xe)
    xc = x.detach().clone().requires_grad_(True)
    lc = compiled(xc)
    (gc,) = torch.autograd.grad(lc, xc)
    torch.testing.assert_close(lc, le, rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(gc, ge, rtol=1e-5, atol=1e-9)


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_hip_graph_replays(binning) -> None:
    """Forward + backward captured in a HIP graph: every replay, with eager
    work and synchronisations between replays, equals the eager result."""
    x, y = _inputs(5)
    cfg = ACEConfig(binning=binning, to_onehot_y=True)
    leaf = x.detach().clone().requires_grad_(True)

    def step():
        (g,) = torch.autograd.grad(ace_loss(leaf, y, cfg, impl="hip_mi355x").sum(), leaf)
        return g

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    say(f"graph capture {binning}")
    with torch.cuda.graph(graph, stream=side):
        g_static = step()
    eager = step().clone()
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_static, eager), f"replay {i}"
        _ = (x * 2).sum().item()  # eager work between replays
        eager2 = step()
        assert torch.equal(eager2, eager)


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_no_host_synchronisation(binning) -> None:
    x, y = _inputs(6)
    cfg = ACEConfig(binning=binning, to_onehot_y=True)
    leaf = x.detach().clone().requires_grad_(True)
    for _ in range(2):  # warm-up: tables, class weights and workspace cached
        torch.autograd.grad(ace_loss(leaf, y, cfg, impl="hip_mi355x").sum(), leaf)
    torch.cuda.synchronize()
    say(f"sync debug {binning}")
    torch.cuda.set_sync_debug_mode("error")
    try:
        (g,) = torch.autograd.grad(ace_loss(leaf, y, cfg, impl="hip_mi355x").sum(), leaf)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    assert torch.isfinite(g).all()


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_kernel_stamped_timing_events(binning) -> None:
    """ace_set_launch_events: the forward and backward kernels stamp two
    events (their elapsed time is positive and at most that of events
    recorded on the stream around the same call), the results do not change,
    and clearing the events restores the plain launch."""
    from ace_kernels import _lib

    x, y = _inputs(7, shape=(2, 4, 32, 32, 32))
    cfg = ACEConfig(binning=binning, to_onehot_y=True)
    leaf = x.detach().clone().requires_grad_(True)

    def step():
        loss = ace_loss(leaf, y, cfg, impl="hip_mi355x")
        (g,) = torch.autograd.grad(loss.sum(), leaf)
        return loss.detach(), g

    want_loss, want_grad = step()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    for e in ev:
        e.record()
    torch.cuda.synchronize()
    say(f"stamped events {binning}")
    ev[0].record()
    try:
        _lib.check(_lib.lib().ace_set_launch_events(ev[1].cuda_event, ev[2].cuda_event),
                   "ace_set_launch_events")
        loss = ace_loss(leaf, y, cfg, impl="hip_mi355x")
    finally:
        _lib.lib().ace_set_launch_events(None, None)
    ev[3].record()
    (g,) = torch.autograd.grad(loss.sum(), leaf)
    torch.cuda.synchronize()
    kernel_ms = ev[1].elapsed_time(ev[2])
    around_ms = ev[0].elapsed_time(ev[3])
    say(f"forward kernel {kernel_ms * 1e3:.1f} us, stream events {around_ms * 1e3:.1f} us")
    assert 0.0 < kernel_ms <= around_ms
    assert torch.equal(loss.detach(), want_loss)
    assert torch.equal(g, want_grad)
    again_loss, again_grad = step()
    assert torch.equal(again_loss, want_loss) and torch.equal(again_grad, want_grad)


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_concurrent_streams(binning) -> None:
    """Forwards and backwards issued on two streams at once use one workspace
    per stream and share no device state: every result equals the one
    computed alone on the default stream."""
    cfg = ACEConfig(binning=binning, to_onehot_y=True)
    inputs = [_inputs(10 + i, shape=(2, 4, 32, 32, 32)) for i in range(2)]
    leaves = [x.detach().clone().requires_grad_(True) for x, _ in inputs]

    def step(i):
        loss = ace_loss(leaves[i], inputs[i][1], cfg, impl="hip_mi355x")
        (g,) = torch.autograd.grad(loss.sum(), leaves[i])
        return loss.detach(), g

    want = [step(i) for i in range(2)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(2)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    say(f"concurrent streams {binning}")
    got = [[], []]
    for _ in range(20):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                got[i].append(step(i))
    torch.cuda.synchronize()
    for i in range(2):
        for loss, g in got[i]:
            assert torch.equal(loss, want[i][0])
            assert torch.equal(g, want[i][1])
