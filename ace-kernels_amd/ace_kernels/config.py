"""Options of the mL1-ACE loss.

Same fields, defaults and validation as the reference's ``ACEConfig``
(``src/ace_kernels/config.py:12-31``): a frozen pydantic model that rejects
unknown keys, so a config written for the reference validates unchanged here.
"""

from __future__ import annotations

from typing import Literal, Optional, Tuple, Union

import torch.utils._pytree
from pydantic import BaseModel, ConfigDict, Field

Binning = Literal["hard", "soft"]
Activation = Literal["softmax", "sigmoid", "none"]
Reduction = Literal["mean", "sum", "none"]


class ACEConfig(BaseModel):
    """Loss options, mirroring ``HardL1ACELoss`` / ``SoftL1ACELoss``.

    binning:              "hard" (one bin per probability) or "soft" (linear
                          interpolation between the two nearest bin centres).
    num_bins:             K >= 1 equal-width bins over [0, 1 + eps32].
    activation:           applied to ``input`` along the channel axis; softmax
                          over a single channel is the identity.
    to_onehot_y:          target holds class indices ``[B, 1, *spatial]``.
    include_background:   False drops channel 0 from the loss (not from softmax).
    ignore_empty_classes: classes absent from the target contribute 0.
    reduction:            over the ``[B, C']`` per-class errors.
    weight:               per-class (or one scalar) loss weight, >= 0.
    right:                bucketize convention (False: edge < p counts).
    empty_weight:         soft binning: a bin with weight below this is empty.
    """

    model_config = ConfigDict(frozen=True, extra="forbid")

    binning: Binning = "hard"
    num_bins: int = Field(default=20, ge=1)
    activation: Activation = "softmax"
    to_onehot_y: bool = False
    include_background: bool = True
    ignore_empty_classes: bool = True
    reduction: Reduction = "mean"
    weight: Optional[Union[Tuple[float, ...], float]] = None
    right: bool = False
    empty_weight: float = Field(default=0.01, ge=0.0)


# torch.compile: an ACEConfig is a constant of the traced program (frozen,
# hashable, compared by value), so `ace_loss(net(x), y, config, impl=...)`
# traces with the config folded in, as the reference's compile test does
# (tests/test_triton.py:474-495 upstream).  Without this, dynamo cannot pass
# the pydantic object to the custom ops' constant JSON argument.
if hasattr(torch.utils._pytree, "register_constant"):
    torch.utils._pytree.register_constant(ACEConfig)
