"""End-to-end training step with the loss: the reference's e2e check
(``src/ace_bench/e2e.py``) without MONAI.

The reference trains MONAI's SegResNetDS (``init_filters`` 32, ``blocks_down``
(1, 2, 2, 4, 4), instance norm, deep-supervision depth 4) under
``DeepSupervisionLoss(weight_mode="exp")`` around 0.33 * (Dice + CE +
mL1-ACE), with AdamW (lr 1e-4, weight decay 1e-5) and fp16 autocast, on
synthetic learnable volumes regenerated from the seed at every step
(``e2e.py:122-193``).  MONAI is not installed here, so this module writes the
pieces in plain torch from their published definitions:

- ``SegResNetDS``: residual blocks (instance norm, ReLU, 3^3 convolution,
  twice, plus the identity), a stride-2 convolution between encoder levels
  (filters doubling), transposed-convolution upsampling with additive skips
  in the decoder, and a 1^3 convolution head on the last ``dsdepth`` decoder
  levels; outputs listed from full resolution down.  Same shape and depth as
  the upstream network, not its exact parameterisation.
- ``DiceLoss`` with ``to_onehot_y``, ``softmax``, ``squared_pred``,
  ``smooth_nr`` 0, ``smooth_dr`` 1e-5, mean over batch and classes.
- ``DeepSupervisionLoss(weight_mode="exp")``: level l weighs
  max(0.5^l, 1/16); each level's target is the label map resized with
  nearest interpolation; the wrapped loss gets float32 logits.

``ace`` selects the mL1-ACE term: an impl name (one ``ace_loss`` call per
level, as the reference's step makes), ``"levels"`` (``ace_loss_levels``:
one launch per direction for every level) or ``"none"`` (Dice + CE only,
the step the ACE term is measured against).

    python -m ace_kernels.e2e --steps 30 --patch 96 --batch 2
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
from dataclasses import asdict, dataclass, field
from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F
from torch import nn

from ace_kernels.config import ACEConfig
from ace_kernels.registry import ace_loss


# ---------------------------------------------------------------- network

class ResBlock(nn.Module):
    """norm -> ReLU -> conv, twice, plus the identity."""

    def __init__(self, channels: int) -> None:
        super().__init__()
        self.norm1 = nn.InstanceNorm3d(channels, affine=True)
        self.conv1 = nn.Conv3d(channels, channels, 3, padding=1, bias=False)
        self.norm2 = nn.InstanceNorm3d(channels, affine=True)
        self.conv2 = nn.Conv3d(channels, channels, 3, padding=1, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = self.conv1(F.relu(self.norm1(x)))
        y = self.conv2(F.relu(self.norm2(y)))
        return x + y


class SegResNetDS(nn.Module):
    """Encoder-decoder with deep-supervision heads (see the module docstring)."""

    def __init__(self, in_channels: int = 1, out_channels: int = 4, init_filters: int = 32,
                 blocks_down: Sequence[int] = (1, 2, 2, 4, 4), dsdepth: int = 4) -> None:
        super().__init__()
        self.conv_init = nn.Conv3d(in_channels, init_filters, 3, padding=1, bias=False)
        self.down_blocks = nn.ModuleList()
        self.downsample = nn.ModuleList()
        filters = init_filters
        for i, n in enumerate(blocks_down):
            self.down_blocks.append(nn.Sequential(*[ResBlock(filters) for _ in range(n)]))
            if i < len(blocks_down) - 1:
                self.downsample.append(nn.Conv3d(filters, 2 * filters, 3, stride=2, padding=1,
                                                 bias=False))
                filters *= 2
        n_up = len(blocks_down) - 1
        self.upsample = nn.ModuleList()
        self.up_blocks = nn.ModuleList()
        self.heads = nn.ModuleDict()
        for i in range(n_up):
            self.upsample.append(nn.ConvTranspose3d(filters, filters // 2, 2, stride=2, bias=False))
            filters //= 2
            self.up_blocks.append(ResBlock(filters))
            if i >= n_up - dsdepth:
                self.heads[str(i)] = nn.Conv3d(filters, out_channels, 1)

    def forward(self, x: torch.Tensor) -> List[torch.Tensor]:
        x = self.conv_init(x)
        skips = []
        for i, blocks in enumerate(self.down_blocks):
            x = blocks(x)
            skips.append(x)
            if i < len(self.downsample):
                x = self.downsample[i](x)
        x = skips.pop()
        outs = []
        for i, (up, blocks) in enumerate(zip(self.upsample, self.up_blocks)):
            x = blocks(up(x) + skips.pop())
            if str(i) in self.heads:
                outs.append(self.heads[str(i)](x))
        return outs[::-1]  # full resolution first


# ---------------------------------------------------------------- losses

def dice_loss(logits: torch.Tensor, labels: torch.Tensor, smooth_nr: float = 0.0,
              smooth_dr: float = 1e-5) -> torch.Tensor:
    """Dice with softmax, one-hot labels and squared predictions, averaged
    over batch and classes."""
    p = torch.softmax(logits, 1)
    y = F.one_hot(labels[:, 0].long(), logits.shape[1]).movedim(-1, 1).to(p.dtype)
    dims = tuple(range(2, logits.dim()))
    inter = (p * y).sum(dims)
    denom = (y * y).sum(dims) + (p * p).sum(dims)
    return (1.0 - (2.0 * inter + smooth_nr) / (denom + smooth_dr)).mean()


def ds_weights(levels: int) -> List[float]:
    return [max(0.5 ** level, 0.0625) for level in range(levels)]


def level_targets(labels: torch.Tensor, outputs: Sequence[torch.Tensor]) -> List[torch.Tensor]:
    """The label map at each output's size (nearest interpolation)."""
    out = []
    for o in outputs:
        if o.shape[2:] == labels.shape[2:]:
            out.append(labels)
        else:
            out.append(F.interpolate(labels, size=o.shape[2:], mode="nearest"))
    return out


@dataclass
class StepLoss:
    """0.33 * (Dice + CE + ACE) per level, weighted over the levels; the ACE
    terms are also kept (weighted sum) for the curves."""

    binning: str
    ace: str  # impl name, "levels" or "none"

    def __post_init__(self) -> None:
        self.config = ACEConfig(binning=self.binning, to_onehot_y=True)

    def __call__(self, outputs: Sequence[torch.Tensor], labels: torch.Tensor):
        weights = ds_weights(len(outputs))
        targets = level_targets(labels, outputs)
        logits = [o.float() for o in outputs]
        aces: List[Optional[torch.Tensor]] = [None] * len(outputs)
        if self.ace == "levels":
            from ace_kernels.levels import ace_loss_levels

            aces = ace_loss_levels(logits, targets, self.config)
        elif self.ace != "none":
            aces = [ace_loss(lg, t, self.config, impl=self.ace) for lg, t in zip(logits, targets)]
        total = logits[0].new_zeros(())
        ace_sum = logits[0].new_zeros(())
        for w, lg, t, a in zip(weights, logits, targets, aces):
            term = dice_loss(lg, t) + F.cross_entropy(lg, t[:, 0].long())
            if a is not None:
                term = term + a
                ace_sum = ace_sum + w * a.detach()
            total = total + w * 0.33 * term
        return total, ace_sum


# ---------------------------------------------------------------- data and step

def synthetic_batch(step: int, seed: int, batch: int, classes: int, patch: Sequence[int],
                    device: str) -> Tuple[torch.Tensor, torch.Tensor]:
    """A smooth random label map and a noisy intensity image, deterministic per
    step (e2e.py:122-137): float labels, as loaded upstream."""
    gen = torch.Generator().manual_seed(seed * 1_000_003 + step)
    coarse = torch.randn(batch, classes, *(max(1, s // 8) for s in patch), generator=gen)
    labels = F.interpolate(coarse, size=tuple(patch), mode="trilinear").argmax(1, keepdim=True)
    noise = torch.randn(batch, 1, *patch, generator=gen)
    image = labels.float() / (classes - 1) + 0.3 * noise
    return image.to(device), labels.float().to(device)


@dataclass
class E2EConfig:
    binning: str = "hard"
    ace: str = "hip_mi355x"
    classes: int = 4
    batch: int = 2
    patch: Tuple[int, int, int] = (96, 96, 96)
    init_filters: int = 32
    steps: int = 30
    skip_steps: int = 5
    lr: float = 1e-4
    amp: bool = True
    seed: int = 0
    device: str = "cuda"


@dataclass
class E2EResult:
    config: dict
    losses: List[float] = field(default_factory=list)
    aces: List[float] = field(default_factory=list)
    step_ms: List[float] = field(default_factory=list)
    peak_mib: Optional[float] = None

    def summary(self) -> dict:
        timed = self.step_ms[self.config["skip_steps"]:] or self.step_ms
        return {
            "config": self.config,
            "step_ms_p50": statistics.median(timed) if timed else None,
            "step_ms_mean": statistics.fmean(timed) if timed else None,
            "loss_first": self.losses[0] if self.losses else None,
            "loss_last": self.losses[-1] if self.losses else None,
            "ace_first": self.aces[0] if self.aces else None,
            "ace_last": self.aces[-1] if self.aces else None,
            "peak_mib": self.peak_mib,
        }


def build(cfg: E2EConfig):
    torch.manual_seed(cfg.seed)
    model = SegResNetDS(1, cfg.classes, cfg.init_filters).to(cfg.device)
    opt = torch.optim.AdamW(model.parameters(), lr=cfg.lr, weight_decay=1e-5)
    return model, opt


def train(cfg: E2EConfig) -> E2EResult:
    """``cfg.steps`` training steps; on a HIP device each is timed with events
    around zero_grad .. scaler.update, as the reference's step."""
    model, opt = build(cfg)
    model.train()
    loss_fn = StepLoss(cfg.binning, cfg.ace)
    cuda = cfg.device.startswith("cuda")
    use_amp = cfg.amp and cuda
    scaler = torch.amp.GradScaler(enabled=use_amp)
    res = E2EResult(config=asdict(cfg))
    if cuda:
        torch.cuda.reset_peak_memory_stats()
    for step in range(cfg.steps):
        image, labels = synthetic_batch(step, cfg.seed, cfg.batch, cfg.classes, cfg.patch,
                                        cfg.device)
        if cuda:
            torch.cuda.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
        opt.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.float16, enabled=use_amp):
            outputs = model(image)
        loss, ace_sum = loss_fn(outputs, labels)
        scaler.scale(loss).backward()
        scaler.step(opt)
        scaler.update()
        if cuda:
            end.record()
            torch.cuda.synchronize()
            res.step_ms.append(start.elapsed_time(end))
        res.losses.append(float(loss.detach()))
        res.aces.append(float(ace_sum))
    if cuda:
        res.peak_mib = torch.cuda.max_memory_allocated() / 2**20
    return res


def main(argv: Optional[List[str]] = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--skip-steps", type=int, default=5)
    ap.add_argument("--patch", type=int, default=96)
    ap.add_argument("--batch", type=int, default=2)
    ap.add_argument("--init-filters", type=int, default=32)
    ap.add_argument("--binnings", default="hard,soft")
    ap.add_argument("--aces", default="none,hip_mi355x,levels")
    args = ap.parse_args(argv)
    for binning in args.binnings.split(","):
        for ace in args.aces.split(","):
            cfg = E2EConfig(binning=binning, ace=ace, batch=args.batch,
                            patch=(args.patch,) * 3, init_filters=args.init_filters,
                            steps=args.steps, skip_steps=args.skip_steps)
            print(f"e2e {binning} ace={ace}: {cfg.steps} steps", file=sys.stderr, flush=True)
            print(json.dumps(train(cfg).summary()), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
