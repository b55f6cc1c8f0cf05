"""Convert the reference's golden file into ``reference_cases.npz`` (data only).

The reference ships ``tests/golden/reference_cases.pt``: 43 cases, each holding
the input, target, ACEConfig, loss and d(loss.sum())/d(input), written by the
reference's own ``scripts/make_golden.py`` on its platform (torch 2.14.1, monai
1.6.1, macOS arm64 CPU).  This script reads that file as data with
``torch.load(..., weights_only=True)`` (no code from the reference runs) and
rewrites it as a plain NumPy archive so the GPU box, which has no copy of the
reference, can load it with ``numpy.load`` (``allow_pickle=False``).

Run from the repository root, in a container where the reference is mounted:

    python tests/golden/make_fixture.py
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

SOURCE = Path("/root/reference/tests/golden/reference_cases.pt")
OUT = Path(__file__).resolve().parent / "reference_cases.npz"


def main() -> None:
    blob = torch.load(SOURCE, weights_only=True)
    arrays = {}
    meta = {"env": blob["env"], "cases": {}}
    for name, rec in sorted(blob["cases"].items()):
        arrays[f"{name}/input"] = rec["input"].numpy()
        arrays[f"{name}/target"] = rec["target"].numpy()
        arrays[f"{name}/loss"] = rec["loss"].numpy()
        arrays[f"{name}/grad"] = rec["grad"].numpy()
        cfg = dict(rec["config"])
        if isinstance(cfg.get("weight"), tuple):
            cfg["weight"] = list(cfg["weight"])
        meta["cases"][name] = cfg
    arrays["__meta__"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {len(meta['cases'])} cases to {OUT} ({OUT.stat().st_size / 1e6:.2f} MB)")


if __name__ == "__main__":
    main()
