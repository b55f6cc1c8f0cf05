"""HIP graphs and the per-stream workspace (ace_kernels.common.workspace).

A captured forward keeps the raw address of the workspace it used.  These
tests run the fixed code paths: the workspace outgrown by a later, larger
eager call on the capture stream is retired, not freed, so replays still
write valid memory; a capture on a stream that has no workspace yet (torch's
default capture stream) gets one of its own, zeroed by the graph itself; and
every replay, with eager work, allocations and synchronisations between
replays, equals the eager result bit for bit."""

from __future__ import annotations

import pytest
import torch

from ace_kernels import ACEConfig, ace_loss
from gpu_helpers import say

pytestmark = pytest.mark.gpu


def _inputs(shape, seed):
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn(shape, generator=gen) * 1.5).cuda()
    y = torch.randint(0, shape[1], (shape[0], 1, *shape[2:]), generator=gen).cuda()
    return x, y


def _step(leaf, y, cfg):
    loss = ace_loss(leaf, y, cfg, impl="hip_mi355x")
    (g,) = torch.autograd.grad(loss.sum(), leaf)
    return loss.detach(), g


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_replay_after_the_workspace_grew(binning) -> None:
    cfg = ACEConfig(binning=binning, to_onehot_y=True, activation="softmax")
    x, y = _inputs((2, 4, 128, 128, 128), 11)  # configuration 2's shape
    leaf = x.clone().requires_grad_(True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    say(f"graph workspace {binning}: warm-up and capture at cfg 2 size")
    with torch.cuda.stream(side):
        for _ in range(2):
            _step(leaf, y, cfg)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        loss_s, g_s = _step(leaf, y, cfg)
    want_loss, want_g = _step(leaf, y, cfg)
    torch.cuda.synchronize()

    # a larger problem eagerly on the capture stream: its workspace grows
    big_x, big_y = _inputs((70, 4, 24, 24, 24), 12)
    big_leaf = big_x.clone().requires_grad_(True)
    say(f"graph workspace {binning}: larger eager problem on the capture stream")
    with torch.cuda.stream(side):
        big_want = _step(big_leaf, big_y, cfg)
    torch.cuda.synchronize()
    for i in range(3):
        # allocations and fills between replays: freed memory would be reused here
        junk = [torch.full((1 << 18,), 7.0 + i, device="cuda") for _ in range(8)]
        with torch.cuda.stream(side):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(loss_s, want_loss), f"replay {i}: loss"
        assert torch.equal(g_s, want_g), f"replay {i}: gradient"
        with torch.cuda.stream(side):
            again = _step(big_leaf, big_y, cfg)
        torch.cuda.synchronize()
        assert torch.equal(again[0], big_want[0]) and torch.equal(again[1], big_want[1])
        del junk


@pytest.mark.parametrize("binning", ["hard", "soft"])
def test_capture_on_a_stream_without_workspace(binning) -> None:
    """torch.cuda.graph's own capture stream, warm-up on another stream."""
    cfg = ACEConfig(binning=binning, to_onehot_y=True, activation="softmax")
    x, y = _inputs((2, 4, 40, 36, 32), 13)
    leaf = x.clone().requires_grad_(True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _step(leaf, y, cfg)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    say(f"graph workspace {binning}: capture on torch's capture stream")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        loss_s, g_s = _step(leaf, y, cfg)
    want = _step(leaf, y, cfg)
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(loss_s, want[0]) and torch.equal(g_s, want[1]), f"replay {i}"
        assert torch.equal(_step(leaf, y, cfg)[1], want[1])
