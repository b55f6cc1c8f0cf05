"""Host-side pieces of the HIP implementation: tables, class weights, workspace.

- Bin tables are part of the loss definition: the reference bins against the
  float32 ``torch.linspace(0, 1 + eps32, K + 1)`` (hard) and
  ``linspace(0, 1 + eps32, 2K + 1)`` (soft) tensors
  (``src/ace_kernels/common.py:17-25``, ``kernels/soft_hist.py:161-170``).
  They are built once per (K, device) by that same library call, on the CPU
  (where the reference and its golden vectors compute them), and copied to the
  device once.  The first call for a new K is therefore not graph-capturable;
  later calls are.
- Class weights are validated on the Python config values exactly as
  ``common.class_weights`` (``common.py:162-181``) and cached on the device.
- The forward's workspace (ticket counters, loss partial words, final sums)
  is cached per (device, stream) and grown on demand; it is zero when created
  and every forward leaves it zero.
"""

from __future__ import annotations

import threading
from functools import lru_cache
from typing import Dict, List, Optional, Tuple

import torch

from ace_kernels.config import ACEConfig

EPS32 = torch.finfo(torch.float32).eps


@lru_cache(maxsize=128)
def bin_tables(num_bins: int, soft: bool, device: torch.device) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """(bucket table, centre table or None) as float32 tensors on ``device``.

    hard: the K upper edges ``linspace(0, 1 + eps32, K + 1)[1:]``;
    soft: the 2K upper half boundaries ``linspace(0, 1 + eps32, 2K + 1)[1:]``
    and the replicated centres ``[-1e4, c0, c0, ..., c_{K-1}, c_{K-1}, 1e4]``.
    """
    if not soft:
        edges = torch.linspace(0.0, 1.0 + EPS32, num_bins + 1)[1:].contiguous()
        return edges.to(device), None
    half = torch.linspace(0.0, 1.0 + EPS32, 2 * num_bins + 1)
    sentinel = torch.full((1,), 10000.0)
    repl = torch.cat((-sentinel, half[1::2].repeat_interleave(2), sentinel))
    return half[1:].contiguous().to(device), repl.contiguous().to(device)


def class_weights(config: ACEConfig, n_ch: int) -> Optional[List[float]]:
    """Per-class loss weights (None: unweighted), validated like the reference."""
    if config.weight is None or n_ch == 1:
        return None
    weights = (
        [float(config.weight)] * n_ch
        if isinstance(config.weight, (int, float))
        else [float(w) for w in config.weight]
    )
    if len(weights) != n_ch:
        raise ValueError(
            "the length of the `weight` sequence should be the same as the "
            "number of classes (excluding background if include_background=False)"
        )
    if min(weights) < 0:
        raise ValueError("the value/values of the `weight` should be no less than 0.")
    return weights


@lru_cache(maxsize=64)
def class_weight_tensor(weights: Tuple[float, ...], device: torch.device) -> torch.Tensor:
    return torch.tensor(weights, dtype=torch.float32, device=device)


_WS_LOCK = threading.Lock()
_WORKSPACES: Dict[Tuple[int, int], list] = {}


def workspace(device: torch.device, stream: int, nbytes: int, reset_bytes: int) -> torch.Tensor:
    """A uint8 device buffer of at least ``nbytes`` for ``stream`` whose first
    ``reset_bytes`` bytes are zero when the next forward on ``stream`` runs.

    One buffer per (device, stream): forwards on one stream are ordered, so
    they share it; forwards on different streams get different buffers.  Every
    forward leaves its reset region (ticket counters, loss partial words and
    final sums) zero, so the leading ``clean`` bytes of the buffer are known
    to be zero, where ``clean`` is the reset size of the last forward; a
    forward that needs more is preceded by one fill of its reset region (only
    when the problem's layout grows).
    """
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    with _WS_LOCK:
        entry = _WORKSPACES.get(key)
        if entry is None or entry[0].numel() < nbytes:
            buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            entry = [buf, buf.numel()]
            _WORKSPACES[key] = entry
        buf, clean = entry
        if reset_bytes > clean:
            buf[:reset_bytes].zero_()
        entry[1] = reset_bytes
        return buf
