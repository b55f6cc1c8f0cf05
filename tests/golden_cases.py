"""Loader for the reference's golden cases (``tests/golden/reference_cases.npz``)."""

from __future__ import annotations

import json
from dataclasses import dataclass
from functools import lru_cache
from pathlib import Path
from typing import Dict

import numpy as np
import torch

PATH = Path(__file__).resolve().parent / "golden" / "reference_cases.npz"


@dataclass(frozen=True)
class GoldenCase:
    name: str
    config: dict
    input: torch.Tensor
    target: torch.Tensor
    loss: torch.Tensor
    grad: torch.Tensor


@lru_cache(maxsize=1)
def load_golden() -> Dict[str, GoldenCase]:
    data = np.load(PATH, allow_pickle=False)
    meta = json.loads(bytes(data["__meta__"]).decode())
    out = {}
    for name, cfg in meta["cases"].items():
        if isinstance(cfg.get("weight"), list):
            cfg["weight"] = tuple(cfg["weight"])
        out[name] = GoldenCase(
            name,
            cfg,
            torch.from_numpy(data[f"{name}/input"].copy()),
            torch.from_numpy(data[f"{name}/target"].copy()),
            torch.from_numpy(data[f"{name}/loss"].copy()),
            torch.from_numpy(data[f"{name}/grad"].copy()),
        )
    return out


def golden_env() -> dict:
    data = np.load(PATH, allow_pickle=False)
    return json.loads(bytes(data["__meta__"]).decode())["env"]
