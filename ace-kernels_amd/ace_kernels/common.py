"""Host-side pieces of the HIP implementation: tables, class weights, workspace.

- Bin tables are part of the loss definition: the reference bins against the
  float32 ``torch.linspace(0, 1 + eps32, K + 1)`` (hard) and
  ``linspace(0, 1 + eps32, 2K + 1)`` (soft) tensors
  (``src/ace_kernels/common.py:17-25``, ``kernels/soft_hist.py:161-170``).
  They are built once per (K, device) by that same library call, on the CPU
  (where the reference and its golden vectors compute them), and copied to the
  device once.
- Class weights are validated on the Python config values exactly as
  ``common.class_weights`` (``common.py:162-181``) and cached on the device.
- The forward's workspace (ticket counters, loss partial words, final sums)
  is cached per (device, stream); it is zero when created and every forward
  leaves it zero.

Every cached device buffer lives until the process ends.  A HIP graph keeps
the raw addresses it captured, so nothing a capture may have used is ever
freed: a table or class-weight tensor is never evicted, and a workspace that
a larger problem outgrows is retired (kept) rather than released.  Tables
and class weights are copied from the host, which a stream capture cannot
record, so the first call of a new (K, device) or class-weight set must run
before capture (inside a capture it raises ``RuntimeError``); a workspace a
capture lacks is made for that capture alone (``workspace``).
"""

from __future__ import annotations

import threading
from typing import Dict, List, Optional, Tuple

import torch

from ace_kernels.config import ACEConfig

EPS32 = torch.finfo(torch.float32).eps

_CACHE_LOCK = threading.Lock()
_TABLES: Dict[Tuple[int, bool, str, int], Tuple[torch.Tensor, Optional[torch.Tensor]]] = {}
_CLASS_WEIGHTS: Dict[Tuple[Tuple[float, ...], str, int, str], torch.Tensor] = {}


def _device_key(device: torch.device) -> Tuple[str, int]:
    device = torch.device(device)
    if device.type == "cuda":
        return "cuda", device.index if device.index is not None else torch.cuda.current_device()
    return device.type, -1 if device.index is None else device.index


def capturing(device: torch.device) -> bool:
    """True while the current stream of ``device`` is being captured."""
    return torch.device(device).type == "cuda" and torch.cuda.is_current_stream_capturing()


def _refuse_under_capture(device: torch.device, what: str) -> None:
    if capturing(device):
        raise RuntimeError(
            f"ace_kernels: {what} does not exist yet and cannot be created during HIP graph "
            "capture (it needs an allocation or a host-to-device copy); run one call of the "
            "same configuration on this stream before capturing"
        )


def bin_tables(num_bins: int, soft: bool, device: torch.device) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """(bucket table, centre table or None) as float32 tensors on ``device``.

    hard: the K upper edges ``linspace(0, 1 + eps32, K + 1)[1:]``;
    soft: the 2K upper half boundaries ``linspace(0, 1 + eps32, 2K + 1)[1:]``
    and the replicated centres ``[-1e4, c0, c0, ..., c_{K-1}, c_{K-1}, 1e4]``.
    Cached for the life of the process.
    """
    key = (int(num_bins), bool(soft), *_device_key(device))
    with _CACHE_LOCK:
        hit = _TABLES.get(key)
        if hit is not None:
            return hit
        _refuse_under_capture(device, f"the bin table for num_bins={num_bins}")
        if not soft:
            edges = torch.linspace(0.0, 1.0 + EPS32, num_bins + 1)[1:].contiguous()
            out: Tuple[torch.Tensor, Optional[torch.Tensor]] = (edges.to(device), None)
        else:
            half = torch.linspace(0.0, 1.0 + EPS32, 2 * num_bins + 1)
            sentinel = torch.full((1,), 10000.0)
            repl = torch.cat((-sentinel, half[1::2].repeat_interleave(2), sentinel))
            out = (half[1:].contiguous().to(device), repl.contiguous().to(device))
        _TABLES[key] = out
        return out


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


def class_weight_tensor(weights: Tuple[float, ...], device: torch.device,
                        dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """The weights as a float32 (or ``dtype``) device tensor, cached for the
    life of the process."""
    key = (tuple(float(w) for w in weights), *_device_key(device), str(dtype))
    with _CACHE_LOCK:
        hit = _CLASS_WEIGHTS.get(key)
        if hit is None:
            _refuse_under_capture(device, "the class-weight tensor")
            hit = torch.tensor(key[0], dtype=dtype, device=device)
            _CLASS_WEIGHTS[key] = hit
        return hit


_WS_LOCK = threading.Lock()
_WORKSPACES: Dict[Tuple[str, int, int], torch.Tensor] = {}
_RETIRED: List[torch.Tensor] = []


def workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """A zeroed uint8 device buffer of at least ``nbytes`` for ``stream``.

    One buffer per (device, stream): calls on one stream are ordered, so they
    share it; calls on different streams get different buffers.  It is zeroed
    (on ``stream``) when created, and every call leaves what it used zero, so
    it is zero whenever a call starts.  When a call needs more, a buffer of
    at least twice the size replaces it; the old one is retired but never
    freed, so a HIP graph that captured it keeps valid memory, used by its
    replays only.  A graph's replays share the capture stream's buffer with
    the eager calls made on that stream until it is replaced: order them
    (replay on the capture stream, or synchronise).

    During a capture on a stream without a large enough buffer, the call gets
    a buffer of its own: allocated from the capture's memory pool, zeroed by
    a fill kernel that the graph records (so every replay starts from zero),
    kept for the life of the process, and never handed to eager calls, whose
    buffer must be zeroed when they run.
    """
    key = (*_device_key(device), int(stream))
    with _WS_LOCK:
        buf = _WORKSPACES.get(key)
        if buf is not None and buf.numel() >= nbytes:
            return buf
        if capturing(device):
            own = torch.zeros(max(int(nbytes), 1), dtype=torch.uint8, device=device)
            _RETIRED.append(own)
            return own
        size = max(int(nbytes), 1 << 16, 2 * (buf.numel() if buf is not None else 0))
        new = torch.zeros(size, dtype=torch.uint8, device=device)
        if buf is not None:
            _RETIRED.append(buf)
        _WORKSPACES[key] = new
        return new
