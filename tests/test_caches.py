"""Host caches of the HIP impl (tables, class weights, workspace): nothing a
HIP graph may have captured is ever freed, tables and class weights are not
created during a capture, and a capture's own workspace stays out of eager
use (CPU tests; the capture state is simulated).  The device-side
regression test is tests/test_gpu_graph_workspace.py."""

from __future__ import annotations

import pytest
import torch

from ace_kernels import common


def test_tables_are_kept_for_the_process() -> None:
    dev = torch.device("cpu")
    a = common.bin_tables(37, True, dev)
    for k in range(1, 300):  # more than any LRU bound would keep
        common.bin_tables(k, False, dev)
    b = common.bin_tables(37, True, dev)
    assert a[0] is b[0] and a[1] is b[1]


def test_class_weights_are_kept_for_the_process() -> None:
    dev = torch.device("cpu")
    w = common.class_weight_tensor((1.0, 2.0, 0.5), dev)
    for k in range(200):
        common.class_weight_tensor((float(k),), dev)
    assert common.class_weight_tensor((1.0, 2.0, 0.5), dev) is w


def test_workspace_grows_and_retires_without_freeing() -> None:
    dev = torch.device("cpu")
    stream = 987654321  # a key of its own
    small = common.workspace(dev, stream, 1000)
    assert small.numel() >= 1000 and int(small.sum()) == 0
    assert common.workspace(dev, stream, 500) is small
    big = common.workspace(dev, stream, small.numel() + 1)
    assert big is not small and big.numel() >= 2 * small.numel()
    assert any(t is small for t in common._RETIRED)  # still referenced: never freed
    assert int(big.sum()) == 0
    assert common.workspace(dev, stream + 1, 10) is not big  # one buffer per stream


def test_nothing_is_created_during_capture(monkeypatch: pytest.MonkeyPatch) -> None:
    dev = torch.device("cpu")
    stream = 192837465
    ws = common.workspace(dev, stream, 4096)
    tab = common.bin_tables(23, False, dev)
    monkeypatch.setattr(common, "capturing", lambda device: True)
    # cached objects are returned as they are
    assert common.workspace(dev, stream, 4096) is ws
    assert common.bin_tables(23, False, dev) is tab
    # a workspace the capture lacks is its own: zeroed, kept for the
    # process, and not the buffer eager calls on that stream get
    own = common.workspace(dev, stream, ws.numel() + 1)
    assert own is not ws and own.numel() > ws.numel() and int(own.sum()) == 0
    assert any(t is own for t in common._RETIRED)
    other = common.workspace(dev, stream + 7, 16)
    monkeypatch.setattr(common, "capturing", lambda device: False)
    assert common.workspace(dev, stream, 4096) is ws
    assert common.workspace(dev, stream + 7, 16) is not other
    monkeypatch.setattr(common, "capturing", lambda device: True)
    # tables and class weights come from the host: a capture cannot record that
    with pytest.raises(RuntimeError, match="graph capture"):
        common.bin_tables(3001, False, dev)
    with pytest.raises(RuntimeError, match="graph capture"):
        common.class_weight_tensor((3.0, 4.0), dev)
