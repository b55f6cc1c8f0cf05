"""Seeded synthetic inputs of the five benchmark configurations.

Each configuration is a loss call on channels-first logits with int64 class
labels (``to_onehot_y=True``, softmax), generated on the CPU with a seeded
``torch.Generator`` and then copied to the device:

1. hard, K=20, x[2,4,64,64,64] ~ N(0, 1.5^2); labels uniform in [0,4);
   +2.0 on the labelled channel for a seeded 70% of voxels (CPU config)
2. hard, K=20, x[2,4,128,128,128] ~ N(0, 1.5^2); labels with class
   frequencies {0.90, 0.06, 0.03, 0.01}; +2.5 on the true class for 80%
3. soft, K=20, the tensors of configuration 2
4. hard, K=20, x[1,16,128,128,128] ~ N(0, 2^2); labels Zipf(s=1.2) over 16
   classes (p_k ~ (k+1)^-1.2); +3.0 on the true class for 75%
5. soft, K=50, bfloat16 x[32,4,512,512] ~ N(0, 1); labels uniform in [0,4);
   +1.5 for 60%; background excluded from the loss

Deep supervision (``deep_supervision(binning)``): the four output levels of
SegResNetDS at a 128^3 patch -- x[1,4,s,s,s] for s = 128, 64, 32, 16, one loss
call per level and one backward through their sum per step (the reference's
``bench/configs/sprint11_deepsup.yaml``, shapes ds0-128 ... ds3-16), with the
distribution of configuration 2.

"N(0, s)" is read with s the standard deviation (``randn * scale``), as the
reference's ``make_inputs`` (``src/ace_kernels/cases.py:60-63``); the bias is
added on the label channel with ``scatter_add`` like ``cases.py:90-93``, under
a Bernoulli mask.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Tuple

import torch

from ace_kernels.config import ACEConfig


@dataclass(frozen=True)
class Workload:
    index: int
    name: str
    batch: int
    channels: int
    spatial: Tuple[int, ...]
    scale: float
    class_probs: Tuple[float, ...]
    bias: float
    bias_fraction: float
    dtype: torch.dtype
    config: ACEConfig
    seed: int = 0

    @property
    def shape(self) -> Tuple[int, ...]:
        return (self.batch, self.channels, *self.spatial)

    @property
    def voxels(self) -> int:
        n = 1
        for s in self.spatial:
            n *= s
        return n

    def input_bytes(self) -> int:
        return self.batch * self.channels * self.voxels * torch.empty((), dtype=self.dtype).element_size()

    def target_bytes(self) -> int:
        return self.batch * self.voxels * 8

    def ideal_bytes(self, mode: str = "fwd_bwd") -> int:
        """Algorithmic bytes (reference ``src/ace_bench/calculator.py:24-27``):
        fwd = x + target; fwd+bwd = 2 (x + target) + x (dx in x's dtype)."""
        xb, tb = self.input_bytes(), self.target_bytes()
        return xb + tb if mode == "fwd" else 2 * (xb + tb) + xb

    def make(self, device: str = "cpu") -> Tuple[torch.Tensor, torch.Tensor]:
        """(logits [B, C, *spatial], labels [B, 1, *spatial] int64) on ``device``."""
        gen = torch.Generator().manual_seed(self.seed)
        x = torch.randn(self.shape, generator=gen) * self.scale
        probs = torch.tensor(self.class_probs, dtype=torch.float64)
        n = self.batch * self.voxels
        labels = torch.multinomial(probs, n, replacement=True, generator=gen)
        labels = labels.view(self.batch, 1, *self.spatial)
        mask = torch.rand(labels.shape, generator=gen) < self.bias_fraction
        x.scatter_add_(1, labels, mask.to(x.dtype) * self.bias)
        return x.to(self.dtype).to(device), labels.to(device)


def _zipf(k: int, s: float) -> Tuple[float, ...]:
    w = [(i + 1) ** -s for i in range(k)]
    total = sum(w)
    return tuple(v / total for v in w)


def _paper(**kw) -> ACEConfig:
    return ACEConfig(to_onehot_y=True, activation="softmax", **kw)


WORKLOADS: Dict[int, Workload] = {
    1: Workload(1, "cfg1-hard-2x4x64^3-fp32", 2, 4, (64, 64, 64), 1.5, (0.25,) * 4, 2.0, 0.70,
                torch.float32, _paper(binning="hard", num_bins=20), seed=1),
    2: Workload(2, "cfg2-hard-2x4x128^3-fp32", 2, 4, (128, 128, 128), 1.5, (0.90, 0.06, 0.03, 0.01),
                2.5, 0.80, torch.float32, _paper(binning="hard", num_bins=20), seed=2),
    3: Workload(3, "cfg3-soft-2x4x128^3-fp32", 2, 4, (128, 128, 128), 1.5, (0.90, 0.06, 0.03, 0.01),
                2.5, 0.80, torch.float32, _paper(binning="soft", num_bins=20), seed=2),
    4: Workload(4, "cfg4-hard-1x16x128^3-fp32", 1, 16, (128, 128, 128), 2.0, _zipf(16, 1.2), 3.0, 0.75,
                torch.float32, _paper(binning="hard", num_bins=20), seed=4),
    5: Workload(5, "cfg5-soft-K50-32x4x512^2-bf16-nobg", 32, 4, (512, 512), 1.0, (0.25,) * 4, 1.5, 0.60,
                torch.bfloat16, _paper(binning="soft", num_bins=50, include_background=False), seed=5),
}


def deep_supervision(binning: str) -> List[Workload]:
    """The four levels of the deep-supervision step (128^3 ... 16^3, B=1, C=4)."""
    out = []
    for level, side in enumerate((128, 64, 32, 16)):
        out.append(Workload(100 + level, f"ds{level}-{side}-{binning}", 1, 4, (side,) * 3, 1.5,
                            (0.90, 0.06, 0.03, 0.01), 2.5, 0.80, torch.float32,
                            _paper(binning=binning, num_bins=20), seed=20 + level))
    return out


def workload(index: int) -> Workload:
    return WORKLOADS[index]


def all_workloads() -> List[Workload]:
    return [WORKLOADS[i] for i in sorted(WORKLOADS)]
