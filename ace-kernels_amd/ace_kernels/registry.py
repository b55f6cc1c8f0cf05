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
    """A registered implementation and the settings it supports."""

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
    """Decorator adding an implementation to the registry under ``name``."""

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
    """Registered implementations, optionally filtered by binning and device."""
    return [
        spec
        for spec in _REGISTRY.values()
        if (binning is None or binning in spec.binnings)
        and (device is None or device in spec.devices)
    ]


def ace_loss(
    input: torch.Tensor,
    target: torch.Tensor,
    config: Optional[ACEConfig] = None,
    impl: str = "reference",
) -> torch.Tensor:
    """Compute the mL1-ACE loss with the chosen implementation.

    Args:
        input: logits or probabilities, shape ``[B, C, *spatial]``.
        target: one-hot ``[B, C, *spatial]``, or labels ``[B, 1, *spatial]``
            when ``config.to_onehot_y`` is set.
        config: loss options; defaults to ``ACEConfig()``.
        impl: registered implementation name. This package registers
            ``"hip_mi355x"``; ``"reference"`` exists only where a CPU reference
            implementation has been registered (the test suite does so).
    """
    config = config if config is not None else ACEConfig()
    spec = get_impl(impl)
    if not spec.supports(config.binning, input.device.type):
        raise ValueError(
            f"{impl!r} does not support binning={config.binning!r} "
            f"on device={input.device.type!r}"
        )
    return spec.fn(input, target, config)
