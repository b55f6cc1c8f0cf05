"""Several levels of one mL1-ACE loss in one launch per direction.

Deep supervision computes the same loss on up to four resolutions of one
batch per step; the reference runs one ``ace_loss`` call per level
(``bench/configs/sprint11_deepsup.yaml``, ``docs/report.md:620-627``), and at
the small levels each call is bound by its launches and cross-block latency.
``ace_loss_levels`` runs every level's forward in one ``ace_forward_levels``
launch and every level's backward in one ``ace_backward_levels`` launch.
Each level's loss and gradient are bit-identical to ``ace_loss(input, target,
config, impl="hip_mi355x")`` on that level alone.

Only configurations with a fast kernel: softmax activation, class-index
targets (``to_onehot_y``), C in {2, 3, 4, 16}, the same batch, channels and
dtype on every level; anything else raises (call ``ace_loss`` per level).

A levels signature (configuration, every level's input and target shapes
and dtypes, device, stream) that has run once, with contiguous inputs that
need no conversion, runs in C++ (``_ace_autograd.ace_loss_levels``: one
forward launch and one backward node for all levels); other calls run the
autograd Function below.
"""

from __future__ import annotations

import ctypes
from typing import Any, Dict, List, Optional, Sequence, Tuple

import torch

from ace_kernels import _lib
from ace_kernels.common import capturing, class_weight_tensor, class_weights, workspace
from ace_kernels.config import ACEConfig
from ace_kernels.impls.hip_mi355x import Plan, _d_shape, _d_values, _ptr, _stream, make_plan, saved_layout

_REDUCTIONS = {"mean": _lib.RED_MEAN, "sum": _lib.RED_SUM, "none": _lib.RED_NONE}
MAX_LEVELS = 4


def _check_plans(plans: Sequence[Plan]) -> None:
    if not 1 <= len(plans) <= MAX_LEVELS:
        raise ValueError(f"ace_loss_levels takes 1 to {MAX_LEVELS} levels, got {len(plans)}")
    p0 = plans[0]
    if p0.dtype_code == _lib.F64:
        raise TypeError("ace_loss_levels takes float32 / bfloat16 / float16 logits; "
                        "call ace_loss per level for float64")
    if p0.act != _lib.ACT_SOFTMAX or p0.target_kind != _lib.TARGET_LABELS_I64:
        raise ValueError("ace_loss_levels needs activation='softmax' with to_onehot_y class labels")
    for p in plans[1:]:
        if (p.B, p.C, p.dtype_code, p.x.device) != (p0.B, p0.C, p0.dtype_code, p0.x.device):
            raise ValueError("every level must have the same batch, channels, dtype and device")


def forward_levels(plans: Sequence[Plan], config: ACEConfig):
    """Per level (loss, coef, d, jac) from one ``ace_forward_levels`` launch."""
    lib = _lib.lib()
    p0 = plans[0]
    dev = p0.x.device
    stream = _stream(dev)
    binning = _lib.SOFT if p0.soft else _lib.HARD
    n = len(plans)
    vox = (ctypes.c_int64 * n)(*[p.N for p in plans])
    nbytes = lib.ace_workspace_bytes_levels(n, vox, p0.B, p0.C, p0.K, binning, p0.dtype_code,
                                            int(p0.include_bg))
    ws = workspace(dev, stream, nbytes)
    reduction = _REDUCTIONS[config.reduction]
    f32 = torch.float32
    bck, bc = p0.B * p0.CL * p0.K, p0.B * p0.CL
    nd = _d_values(p0)
    outs = []
    keep = []  # buffers the launch writes that the caller does not get back
    arr = (_lib.AceFwdLevel * n)()
    for i, p in enumerate(plans):
        saved = torch.empty(bck + nd + bc, dtype=f32, device=dev)
        coef = saved[:bck].view(p.B, p.CL, p.K)
        d = saved[bck:bck + nd].view(_d_shape(p))
        jac = saved[bck + nd:].view(p.B, p.CL)
        per_class = torch.empty((p.B, p.CL), dtype=f32, device=dev)
        keep.append(per_class)
        loss = torch.empty((), dtype=f32, device=dev) if reduction != _lib.RED_NONE else None
        arr[i] = _lib.AceFwdLevel(p.x.data_ptr(), p.target.data_ptr(), p.N, coef.data_ptr(),
                                  d.data_ptr(), jac.data_ptr(), per_class.data_ptr(), _ptr(loss))
        if loss is None:
            loss = per_class.view(p.B, p.CL, *([1] * p.spatial_ndim))
        outs.append((loss, coef, d, jac))
    weights = class_weights(config, p0.CL)
    cw = class_weight_tensor(tuple(weights), dev) if weights is not None else None
    rc = lib.ace_forward_levels(
        n, arr, p0.dtype_code, p0.B, p0.C, p0.K, binning, int(p0.include_bg),
        int(config.ignore_empty_classes), reduction, int(p0.right), float(config.empty_weight),
        _ptr(cw), p0.btab.data_ptr(), _ptr(p0.rtab), ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "ace_forward_levels")
    # freed only now, after the launch was queued: the allocator reuses them
    # in stream order
    del keep
    return outs


def backward_levels(plans: Sequence[Plan], saved, grad_outputs) -> List[torch.Tensor]:
    """Per level d loss / d input from one ``ace_backward_levels`` launch."""
    lib = _lib.lib()
    p0 = plans[0]
    dev = p0.x.device
    n = len(plans)
    per_class = grad_outputs[0].dim() > 0
    arr = (_lib.AceBwdLevel * n)()
    keep, dxs = [], []
    for i, (p, (coef, d, jac), go) in enumerate(zip(plans, saved, grad_outputs)):
        go = go.float() if go.dtype != torch.float32 else go
        go = (go.reshape(-1) if per_class else go.reshape(())).contiguous()
        dx = torch.empty_like(p.x)
        keep.append(go)
        dxs.append(dx)
        arr[i] = _lib.AceBwdLevel(p.x.data_ptr(), p.target.data_ptr() if p.soft else None, p.N,
                                  coef.data_ptr(), d.data_ptr(), jac.data_ptr(), go.data_ptr(),
                                  dx.data_ptr())
    rc = lib.ace_backward_levels(
        n, arr, p0.dtype_code, p0.B, p0.C, p0.K, _lib.SOFT if p0.soft else _lib.HARD,
        int(p0.include_bg), int(p0.right), int(per_class), p0.btab.data_ptr(), _ptr(p0.rtab),
        _stream(dev))
    _lib.check(rc, "ace_backward_levels")
    return [dx.view(p.in_shape) for dx, p in zip(dxs, plans)]


class _HipLevelsLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, config: ACEConfig, n: int, *tensors: torch.Tensor) -> Tuple[torch.Tensor, ...]:
        plans = [make_plan(tensors[i], tensors[n + i], config) for i in range(n)]
        _check_plans(plans)
        outs = forward_levels(plans, config)
        flat = []
        for p, (_, coef, d, jac) in zip(plans, outs):
            flat += [p.x, p.target, coef, d, jac]
            p.x = p.target = None
        ctx.save_for_backward(*flat)
        ctx.plans = plans
        return tuple(o[0] for o in outs)

    @staticmethod
    def backward(ctx: Any, *grads: Optional[torch.Tensor]):
        saved = ctx.saved_tensors
        plans = ctx.plans
        n = len(plans)
        ref = next(g for g in grads if g is not None)
        gos = [g if g is not None else torch.zeros_like(ref) for g in grads]
        for i, p in enumerate(plans):
            p.x, p.target = saved[5 * i], saved[5 * i + 1]
        try:
            dxs = backward_levels(plans, [saved[5 * i + 2:5 * i + 5] for i in range(n)], gos)
        finally:
            for p in plans:
                p.x = p.target = None
        return (None, None, *dxs, *([None] * n))


def _level_signature(plans: Sequence[Plan], config: ACEConfig, stream: int):
    """The C++ levels call's fixed arguments (``_ace_autograd.LevelSignature``)
    and the buffers they point into (kept alive beside it)."""
    lib = _lib.lib()
    p0 = plans[0]
    dev = p0.x.device
    binning = _lib.SOFT if p0.soft else _lib.HARD
    n = len(plans)
    vox = (ctypes.c_int64 * n)(*[p.N for p in plans])
    nbytes = lib.ace_workspace_bytes_levels(n, vox, p0.B, p0.C, p0.K, binning, p0.dtype_code,
                                            int(p0.include_bg))
    ws = workspace(dev, stream, nbytes)
    weights = class_weights(config, p0.CL)
    cw = class_weight_tensor(tuple(weights), dev) if weights is not None else None
    reduction = _REDUCTIONS[config.reduction]
    reduced = reduction != _lib.RED_NONE
    sig = _lib.autograd().make_level_signature(
        p0.dtype_code, p0.B, p0.C, p0.K, binning, int(p0.include_bg), int(config.ignore_empty_classes),
        reduction, int(p0.right), float(config.empty_weight), _ptr(cw) or 0, p0.btab.data_ptr(),
        _ptr(p0.rtab) or 0, ws.data_ptr(), ws.numel(), [p.N for p in plans],
        *saved_layout(p0, reduced), reduced, p0.soft,
        [] if reduced else [p0.B, p0.CL, *([1] * p0.spatial_ndim)])
    return sig, (ws, cw, p0.btab, p0.rtab)


# levels signature -> (LevelSignature, kept buffers), or None for the
# general path; bounded, cleared when full
_LEVEL_CALLS: Dict[Tuple[Any, ...], Optional[Tuple[Any, Tuple[Any, ...]]]] = {}
_MAX_LEVEL_CALLS = 64


def ace_loss_levels(inputs: Sequence[torch.Tensor], targets: Sequence[torch.Tensor],
                    config: ACEConfig) -> List[torch.Tensor]:
    """The loss of each level (same as ``ace_loss(inputs[i], targets[i], config)``)
    from one forward launch; their backward is one launch too."""
    if len(inputs) != len(targets):
        raise ValueError("one target per input")
    n = len(inputs)
    if n == 0:
        raise ValueError(f"ace_loss_levels takes 1 to {MAX_LEVELS} levels, got 0")
    x0 = inputs[0]
    stream = _stream(x0.device) if x0.is_cuda else 0
    key = (config, stream, x0.get_device(),
           *[(x.shape, x.dtype, t.shape, t.dtype, t.get_device()) for x, t in zip(inputs, targets)])
    hit = _LEVEL_CALLS.get(key)
    if hit is not None and all(x.is_contiguous() for x in inputs) and all(t.is_contiguous() for t in targets):
        return _lib.autograd().ace_loss_levels(list(inputs), list(targets), hit[0])
    losses = list(_HipLevelsLoss.apply(config, n, *inputs, *targets))
    if key not in _LEVEL_CALLS and not capturing(x0.device):
        plans = [make_plan(x, t, config) for x, t in zip(inputs, targets)]
        own = all(p.x.data_ptr() == x.data_ptr() and p.x.dtype == x.dtype and x.is_contiguous()
                  and p.target.data_ptr() == t.data_ptr() and p.target.dtype == t.dtype
                  and t.is_contiguous() for p, x, t in zip(plans, inputs, targets))
        if len(_LEVEL_CALLS) >= _MAX_LEVEL_CALLS:
            _LEVEL_CALLS.clear()
        _LEVEL_CALLS[key] = _level_signature(plans, config, stream) if own else None
    return losses
