"""Registry of mL1-ACE implementations and the ``ace_loss`` dispatcher.

Same contract as the reference registry (``src/ace_kernels/registry.py:14-100``):
every implementation is ``fn(input, target, config) -> loss``; ``register``
refuses duplicates with ``ValueError``; ``get_impl`` raises ``KeyError`` for an
unknown name; ``ace_loss`` raises ``ValueError`` when the implementation does not
support the requested binning on the input's device.

PyTorch-ROCm reports HIP devices as ``"cuda"``, so the HIP implementation
registers with ``devices={"cuda"}``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Dict, FrozenSet, List, Optional

import torch

from ace_kernels.config import ACEConfig, Binning

ACEFn = Callable[[torch.Tensor, torch.Tensor, ACEConfig], torch.Tensor]

ALL_BINNINGS: FrozenSet[str] = frozenset({"hard", "soft"})
ALL_DEVICES: FrozenSet[str] = frozenset({"cpu", "cuda"})


@dataclass(frozen=True)
class ImplSpec:
    """One registry entry: the loss function under ``name``, the binnings and
    device types it accepts, a one-line description, and whether it is slow."""

    name: str
    fn: ACEFn
    binnings: FrozenSet[str]
    devices: FrozenSet[str]
    description: str
    slow: bool = False

    def supports(self, binning: Binning, device: str) -> bool:
        return binning in self.binnings and device in self.devices


_REGISTRY: Dict[str, ImplSpec] = {}


def register(
    name: str,
    *,
    description: str,
    binnings: FrozenSet[str] = ALL_BINNINGS,
    devices: FrozenSet[str] = ALL_DEVICES,
    slow: bool = False,
) -> Callable[[ACEFn], ACEFn]:
    """Returns a decorator that files ``fn`` under ``name`` (``ValueError`` if
    the name is taken) and hands ``fn`` back unchanged."""

    def decorator(fn: ACEFn) -> ACEFn:
        if name in _REGISTRY:
            raise ValueError(f"implementation {name!r} already registered")
        _REGISTRY[name] = ImplSpec(name, fn, binnings, devices, description, slow)
        return fn

    return decorator


def get_impl(name: str) -> ImplSpec:
    try:
        return _REGISTRY[name]
    except KeyError:
        raise KeyError(
            f"unknown implementation {name!r}; available: {sorted(_REGISTRY)}"
        ) from None


def available_impls(
    binning: Optional[Binning] = None, device: Optional[str] = None
) -> List[ImplSpec]:
    """Every registry entry, or only those accepting ``binning`` and/or
    ``device`` when given, in registration order."""
    return [
        spec
        for spec in _REGISTRY.values()
        if (binning is None or binning in spec.binnings)
        and (device is None or device in spec.devices)
    ]


def resolve_impl(impl: str, binning: str, device_type: str) -> str:
    """``impl`` itself, or for ``"auto"``: the HIP kernels (``hip_mi355x``) for
    HIP tensors, else the first registered entry accepting ``binning`` on
    ``device_type`` (this package registers none for the CPU)."""
    if impl != "auto":
        return impl
    if device_type == "cuda" and "hip_mi355x" in _REGISTRY:
        return "hip_mi355x"
    for spec in _REGISTRY.values():
        if spec.supports(binning, device_type):
            return spec.name
    raise ValueError(
        f"no registered implementation accepts binning={binning!r} on {device_type!r} tensors "
        "(this package computes on HIP devices; pass tensors on 'cuda')"
    )


def ace_loss(
    input: torch.Tensor,
    target: torch.Tensor,
    config: Optional[ACEConfig] = None,
    impl: str = "auto",
) -> torch.Tensor:
    """The mL1-ACE loss of ``input`` against ``target`` from registry entry ``impl``.

    ``input`` holds ``[B, C, *spatial]`` logits (probabilities when
    ``config.activation`` is "none"); ``target`` holds class ids
    ``[B, 1, *spatial]`` when ``config.to_onehot_y`` is set, per-channel
    targets ``[B, C, *spatial]`` otherwise.  ``config`` defaults to
    ``ACEConfig()``.  ``impl="auto"`` picks ``hip_mi355x`` for HIP tensors
    (``resolve_impl``); any registered name can be given instead.  The
    reference's default name, ``"reference"``, exists only where a CPU
    reference has been registered (the test suite registers its oracle).
    """
    config = config if config is not None else ACEConfig()
    name = resolve_impl(impl, config.binning, input.device.type)
    spec = get_impl(name)
    if not spec.supports(config.binning, input.device.type):
        raise ValueError(
            f"{name!r} does not support binning={config.binning!r} "
            f"on device={input.device.type!r}"
        )
    return spec.fn(input, target, config)
