"""The reference-side ctypes binding that the repository's integration notes
print in their section 3 (the first python block there, read from the file
named by ``DOC``).

The block is executed as written, with the reference helpers it imports
replaced by restatements of their layouts (the reference package itself is
never imported):

- ``edge_table(K, dev)``: ``hard_edges(K, dev).contiguous()`` -- the K upper
  edges ``linspace(0, 1 + eps32, K + 1)[1:]`` (``src/ace_kernels/kernels/
  bins.py:92-95``, ``common.py:17-20``);
- ``soft_tables(K, dev)``: ``(half, repl)`` with ``half`` the full
  ``soft_half_boundaries`` tensor, 2K + 1 values, 0.0 first, and ``repl`` the
  2K + 2 replicated centres (``kernels/soft_hist.py:161-170``,
  ``common.py:23-25``);
- ``as_kernel_input`` (``kernels/act.py:69-73``) and ``_kernel_target``
  (``impls/v5_triton.py:25-32``).

CPU: the tables the block passes to the C-ABI must equal, bit for bit and
in length, the ones this repository's impl passes (``common.bin_tables``,
pinned by the golden cases).  GPU: the block's registered function runs the
golden cases against the reference's stored loss and gradient.
"""

from __future__ import annotations

import re
import sys
import types
from pathlib import Path

import pytest
import torch

from ace_kernels import _lib
from ace_kernels.common import bin_tables
from ace_kernels.common import class_weights as _class_weights
from ace_kernels.config import ACEConfig

DOC = Path(__file__).resolve().parents[1] / "INTEGRATION.md"
EPS32 = torch.finfo(torch.float32).eps


def _binding_source() -> str:
    text = DOC.read_text()
    section = text.split("## 3.", 1)[1].split("\n## 4.", 1)[0]
    blocks = re.findall(r"```python\n(.*?)```", section, flags=re.S)
    assert blocks, f"{DOC.name} section 3 has no python block"
    return blocks[0]


# ---- restated layouts of the reference helpers the block imports

def _edge_table(num_bins: int, device) -> torch.Tensor:
    return torch.linspace(0.0, 1.0 + EPS32, num_bins + 1, device=device)[1:].contiguous()


def _soft_tables(num_bins: int, device):
    half = torch.linspace(0.0, 1.0 + EPS32, 2 * num_bins + 1, device=device).contiguous()
    sentinel = half.new_full((1,), 10000.0)
    repl = torch.cat((-sentinel, half[1::2].repeat_interleave(2), sentinel))
    return half, repl.contiguous()


def _as_kernel_input(x: torch.Tensor) -> torch.Tensor:
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        x = x.float()
    return x.reshape(x.shape[0], x.shape[1], -1).contiguous()


def _kernel_target(target: torch.Tensor, config: ACEConfig, channels: int) -> torch.Tensor:
    b = target.shape[0]
    if config.to_onehot_y and channels > 1:
        return target.reshape(b, -1).long().contiguous()
    return target.reshape(b, channels, -1).contiguous()


def load_binding(monkeypatch) -> dict:
    """Executes the block with stub modules under the reference's names."""
    registered = {}

    def register(name, *, description, binnings=None, devices=None, slow=False):
        def deco(fn):
            registered[name] = fn
            return fn
        return deco

    mods = {
        "ace_kernels.common": {"class_weights": _class_weights},
        "ace_kernels.config": {"ACEConfig": ACEConfig},
        "ace_kernels.kernels": {},
        "ace_kernels.kernels.act": {"as_kernel_input": _as_kernel_input},
        "ace_kernels.kernels.bins": {"edge_table": _edge_table},
        "ace_kernels.kernels.soft_hist": {"soft_tables": _soft_tables},
        "ace_kernels.impls": {},
        "ace_kernels.impls.v5_triton": {"_kernel_target": _kernel_target},
        "ace_kernels.registry": {"register": register},
    }
    for name, attrs in mods.items():
        mod = types.ModuleType(name)
        mod.__dict__.update(attrs)
        monkeypatch.setitem(sys.modules, name, mod)
    monkeypatch.setenv("ACE_HIP_LIB", str(_lib.LIB_PATH))
    ns: dict = {"__name__": "reference_binding"}
    exec(compile(_binding_source(), f"{DOC.name}#3", "exec"), ns)
    ns["__registered__"] = registered
    return ns


@pytest.mark.parametrize("binning", ["hard", "soft"])
@pytest.mark.parametrize("num_bins", [1, 20, 50])
def test_binding_passes_the_abi_tables(monkeypatch, binning: str, num_bins: int) -> None:
    ns = load_binding(monkeypatch)
    assert "hip_mi355x" in ns["__registered__"]
    cfg = ACEConfig(binning=binning, num_bins=num_bins, to_onehot_y=True)
    x = torch.randn(2, 4, 3, 5)
    y = torch.randint(0, 4, (2, 1, 3, 5))
    _, _, kind, b, c, n, soft, inc_bg, btab, rtab = ns["_args"](x, y, cfg)
    want_b, want_r = bin_tables(num_bins, binning == "soft", torch.device("cpu"))
    assert (kind, b, c, n, soft, inc_bg) == (0, 2, 4, 15, int(binning == "soft"), 1)
    assert btab.dtype == torch.float32 and btab.is_contiguous()
    assert btab.numel() == want_b.numel() == (2 * num_bins if binning == "soft" else num_bins)
    assert torch.equal(btab, want_b)
    if binning == "soft":
        assert rtab is not None and torch.equal(rtab, want_r)
    else:
        assert rtab is None and want_r is None


def test_binding_would_catch_the_full_half_table(monkeypatch) -> None:
    """The full 2K + 1 half table (leading 0) is what the block must not
    pass: it differs in length and shifts every half-bin by one."""
    half, _ = _soft_tables(20, "cpu")
    want, _ = bin_tables(20, True, torch.device("cpu"))
    assert half.numel() == want.numel() + 1
    assert not torch.equal(half[:-1], want)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["paper-3d-hard", "paper-3d-soft"])
def test_binding_runs_golden_cases_on_the_device(monkeypatch, name: str) -> None:
    from golden_cases import load_golden

    ns = load_binding(monkeypatch)
    fn = ns["__registered__"]["hip_mi355x"]
    case = load_golden()[name]
    cfg = ACEConfig(**case.config)
    x = case.input.cuda().requires_grad_(True)
    loss = fn(x, case.target.cuda(), cfg)
    (grad,) = torch.autograd.grad(loss.sum(), x)
    torch.testing.assert_close(loss.detach().cpu(), case.loss, rtol=1e-5, atol=1e-7)
    torch.testing.assert_close(grad.cpu(), case.grad, rtol=1e-4, atol=1e-7)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["paper-3d-hard", "paper-3d-soft"])
def test_binding_runs_float64_on_the_device(monkeypatch, name: str) -> None:
    """The binding's float64 route (ace_forward_f64 / ace_backward_f64)
    against the oracle's float64 restatement of the reference's route."""
    from golden_cases import load_golden
    from oracle.v2 import v2_ace

    ns = load_binding(monkeypatch)
    fn = ns["__registered__"]["hip_mi355x"]
    case = load_golden()[name]
    cfg = ACEConfig(**case.config)
    x64 = case.input.double()
    x = x64.cuda().requires_grad_(True)
    loss = fn(x, case.target.cuda(), cfg)
    assert loss.dtype == torch.float64
    (grad,) = torch.autograd.grad(loss.sum(), x)
    leaf = x64.clone().requires_grad_(True)
    want = v2_ace(leaf, case.target, cfg)
    (want_grad,) = torch.autograd.grad(want.sum(), leaf)
    torch.testing.assert_close(loss.detach().cpu(), want.detach(), rtol=1e-10, atol=1e-13)
    torch.testing.assert_close(grad.cpu(), want_grad, rtol=1e-9, atol=1e-13)
