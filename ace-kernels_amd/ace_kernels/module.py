"""Drop-in ``HardL1ACELoss`` / ``SoftL1ACELoss`` modules over the registry.

Same constructor (argument names, order, defaults, validation) and
``forward(input, target)`` as the reference's drop-in classes
(``src/ace_kernels/module.py:24-178``, themselves the upstream losses'
signature), so switching is one import::

    from ace_kernels.module import HardL1ACELoss

Keyword-only ``impl``: ``"auto"`` (default) runs ``hip_mi355x`` for HIP
("cuda") tensors; any registered name (``ace_kernels.available_impls()``) can
be forced.  ``impl="hip_mi355x_op"`` calls the ``torch.library`` custom ops
with the config's JSON text, so a module used inside
``torch.compile(fullgraph=True)`` traces without graph breaks.  This package
has no CPU implementation: ``"auto"`` on a CPU tensor raises ``ValueError``
(the reference falls back to its PyTorch ``v2_recompute`` there).  ``reduction`` accepts "mean" / "sum" / "none" or any
enum whose ``.value`` is one of them (MONAI's ``LossReduction``), without
depending on MONAI.
"""

from __future__ import annotations

from typing import Callable, Optional, Sequence, Tuple, Union

import torch

from ace_kernels.config import ACEConfig
from ace_kernels.registry import get_impl

FAST_HIP = "hip_mi355x"

Weight = Union[Sequence[float], float, int, torch.Tensor, None]
_REDUCTIONS = ("mean", "sum", "none")


def _reduction(reduction) -> str:
    value = getattr(reduction, "value", reduction)
    if value not in _REDUCTIONS:
        raise ValueError(f"Unsupported reduction: {reduction}, available options are {list(_REDUCTIONS)}.")
    return value


def _config_weight(weight: Weight) -> Union[Tuple[float, ...], float, None]:
    """``weight`` as the plain floats ``ACEConfig.weight`` holds: a 0-d tensor
    or a number becomes one float, a tensor or sequence a tuple of floats."""
    if isinstance(weight, torch.Tensor):
        flat = [float(v) for v in weight.detach().reshape(-1).tolist()]
        return flat[0] if weight.dim() == 0 else tuple(flat)
    if weight is None or isinstance(weight, float):
        return weight
    if isinstance(weight, int):
        return float(weight)
    return tuple(map(float, weight))


class _ACELoss(torch.nn.modules.loss._Loss):
    binning = "hard"

    def __init__(
        self,
        *,
        num_bins: int,
        include_background: bool,
        to_onehot_y: bool,
        sigmoid: bool,
        softmax: bool,
        other_act: Optional[Callable[[torch.Tensor], torch.Tensor]],
        reduction,
        weight: Weight,
        empty_weight: float,
        right: bool,
        ignore_empty_classes: bool,
        impl: str,
    ) -> None:
        red = _reduction(reduction)
        super().__init__(reduction=red)
        if other_act is not None and not callable(other_act):
            raise TypeError(f"other_act must be None or callable but is {type(other_act).__name__}.")
        if int(sigmoid) + int(softmax) + int(other_act is not None) > 1:
            raise ValueError(
                "Incompatible values: more than 1 of [sigmoid=True, softmax=True, other_act is not None]."
            )
        activation = "sigmoid" if sigmoid else "softmax" if softmax else "none"
        self.other_act = other_act
        self.impl = impl
        self.config = ACEConfig(
            binning=self.binning,
            num_bins=num_bins,
            activation=activation,
            to_onehot_y=to_onehot_y,
            include_background=include_background,
            ignore_empty_classes=ignore_empty_classes,
            reduction=red,
            weight=_config_weight(weight),
            right=right,
            empty_weight=empty_weight,
        )
        self.config_json = self.config.model_dump_json()
        if impl != "auto":
            get_impl(impl)  # an unknown name raises KeyError here, at construction

    def resolve_impl(self, device: torch.device) -> str:
        """The registry name this module calls for tensors on ``device``:
        its fixed ``impl``, or with ``"auto"`` the HIP kernels for HIP tensors."""
        if self.impl != "auto":
            return self.impl
        if device.type == "cuda":
            return FAST_HIP
        raise ValueError(
            f"no implementation of this package runs on {device.type!r} tensors; "
            "pass HIP tensors (device 'cuda') or name an implementation with impl="
        )

    def forward(self, input: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
        """Loss of ``input`` (``[B, C, *spatial]`` logits, or probabilities
        when no activation is set) against ``target`` (class ids
        ``[B, 1, *spatial]`` when ``to_onehot_y``, else per-channel targets
        ``[B, C, *spatial]``)."""
        if self.other_act is not None:
            input = self.other_act(input)
        name = self.resolve_impl(input.device)
        if name == "hip_mi355x_op" and input.device.type == "cuda":
            # the custom ops with the JSON text of the config: traceable by
            # torch.compile(fullgraph=True)
            from ace_kernels.impls.hip_mi355x import hip_ace_op_json

            return hip_ace_op_json(input, target, self.config_json)
        spec = get_impl(name)
        if not spec.supports(self.config.binning, input.device.type):
            raise ValueError(
                f"implementation {spec.name!r} does not support binning={self.config.binning!r} "
                f"on device={input.device.type!r}"
            )
        loss: torch.Tensor = spec.fn(input, target, self.config)
        return loss


class HardL1ACELoss(_ACELoss):
    """mL1-ACE with hard binning: each probability counts in the one bin that
    holds it.  Constructor arguments as the upstream class."""

    binning = "hard"

    def __init__(
        self,
        num_bins: int = 20,
        include_background: bool = True,
        to_onehot_y: bool = False,
        sigmoid: bool = False,
        softmax: bool = False,
        other_act: Optional[Callable[[torch.Tensor], torch.Tensor]] = None,
        reduction="mean",
        weight: Weight = None,
        right: bool = False,
        ignore_empty_classes: bool = True,
        *,
        impl: str = "auto",
    ) -> None:
        super().__init__(
            num_bins=num_bins,
            include_background=include_background,
            to_onehot_y=to_onehot_y,
            sigmoid=sigmoid,
            softmax=softmax,
            other_act=other_act,
            reduction=reduction,
            weight=weight,
            empty_weight=0.01,  # the config's default; hard binning never reads it
            right=right,
            ignore_empty_classes=ignore_empty_classes,
            impl=impl,
        )


class SoftL1ACELoss(_ACELoss):
    """mL1-ACE with soft binning: each probability is split between the two
    nearest bin centres.  Constructor arguments as the upstream class."""

    binning = "soft"

    def __init__(
        self,
        num_bins: int = 20,
        include_background: bool = True,
        to_onehot_y: bool = False,
        sigmoid: bool = False,
        softmax: bool = False,
        other_act: Optional[Callable[[torch.Tensor], torch.Tensor]] = None,
        reduction="mean",
        weight: Weight = None,
        empty_weight: float = 0.01,
        right: bool = False,
        ignore_empty_classes: bool = True,
        *,
        impl: str = "auto",
    ) -> None:
        super().__init__(
            num_bins=num_bins,
            include_background=include_background,
            to_onehot_y=to_onehot_y,
            sigmoid=sigmoid,
            softmax=softmax,
            other_act=other_act,
            reduction=reduction,
            weight=weight,
            empty_weight=empty_weight,
            right=right,
            ignore_empty_classes=ignore_empty_classes,
            impl=impl,
        )
