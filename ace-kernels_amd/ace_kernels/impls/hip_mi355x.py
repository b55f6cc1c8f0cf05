"""The MI355X implementation: ``torch.autograd.Function`` over the HIP C-ABI.

Mirrors the reference's fastest implementation, ``_V6Loss``
(``src/ace_kernels/impls/v6_triton.py:93-111``, with ``_forward`` ``:43-65``
and ``_backward`` ``:68-90``): logits in (float32 / bfloat16 / float16),
d logits out in the logits' dtype; saved for backward are the inputs
(already held by the caller) plus ``coef`` ``[B, C', K]``, ``d`` (``[B, C',
K]``; soft binning ``[2, B, C', K]``, d rounded to float32 and its
remainder) and ``jac`` ``[B, C']``.  The forward is one kernel launch
(histograms, cross-block reduction and epilogue); the backward is one
launch.

Input handling follows ``as_kernel_input`` (``kernels/act.py:69-73``) and
``_kernel_target`` (``impls/v5_triton.py:25-32``): logits are viewed as
``[B, C, N]``; with ``to_onehot_y`` and C > 1 the target is read as ``[B, N]``
int64 class indices (one-hot conversion fused into the kernels), else as
``[B, C, N]`` float32 targets.  Errors mirror the reference: a bad input rank
raises ``ValueError`` (``common.py:104-105``), a target/input shape mismatch
``AssertionError`` (``common.py:117-118``), bad class weights ``ValueError``.

float64 input runs the float64 kernels (``ace_forward_f64`` /
``ace_backward_f64``), which compute everything in double with float64
outputs -- the reference sends float64 to its handwritten "recompute"
backward in torch (``v6_triton.py:226-227``); this package has no non-HIP
path.  Their targets are int64 class indices or a float64 one-hot.
"""

from __future__ import annotations

from functools import lru_cache
from typing import Any, Dict, Optional, Tuple

import torch

from ace_kernels import _lib
from ace_kernels.common import bin_tables, capturing, class_weight_tensor, class_weights, workspace
from ace_kernels.config import ACEConfig
from ace_kernels.registry import register

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16,
           torch.float64: _lib.F64}
_REDUCTIONS = {"mean": _lib.RED_MEAN, "sum": _lib.RED_SUM, "none": _lib.RED_NONE}


class Plan:
    """Kernel-ready views of one call's inputs plus the scalar arguments."""

    __slots__ = (
        "x", "dtype_code", "target", "target_kind", "B", "C", "N", "CL", "K",
        "soft", "act", "include_bg", "right", "spatial_ndim", "in_shape",
        "btab", "rtab",
    )


def _activation_code(config: ACEConfig, channels: int) -> int:
    """Softmax over one channel is the identity, as in the reference."""
    if config.activation == "sigmoid":
        return _lib.ACT_SIGMOID
    if config.activation == "softmax" and channels > 1:
        return _lib.ACT_SOFTMAX
    return _lib.ACT_NONE


def make_plan(input: torch.Tensor, target: torch.Tensor, config: ACEConfig) -> Plan:
    if input.dim() < 3:
        raise ValueError(f"input must be [B, C, *spatial], got {tuple(input.shape)}")
    if input.device.type != "cuda":
        raise ValueError(f"hip_mi355x needs a HIP ('cuda') tensor, got {input.device}")
    code = _DTYPES.get(input.dtype)
    x = input if code is not None else input.float()
    code = _DTYPES[x.dtype]
    b, c = x.shape[:2]
    x = x.reshape(b, c, -1)
    if not x.is_contiguous():
        x = x.contiguous()
    n = x.shape[2]
    pl = Plan()
    pl.x, pl.dtype_code = x, code
    pl.B, pl.C, pl.N = int(b), int(c), int(n)
    pl.include_bg = bool(config.include_background or c == 1)
    pl.CL = pl.C - (0 if pl.include_bg else 1)
    pl.K = int(config.num_bins)
    pl.soft = config.binning == "soft"
    pl.act = _activation_code(config, c)
    pl.right = bool(config.right)
    pl.spatial_ndim = input.dim() - 2
    pl.in_shape = input.shape
    if target.device != input.device:
        raise ValueError(f"target is on {target.device}, input on {input.device}")
    if config.to_onehot_y and c > 1:
        t = target.reshape(b, -1)
        if t.shape[1] != n:
            raise AssertionError("target and input spatial sizes differ")
        if t.dtype != torch.int64:
            t = t.long()
        pl.target, pl.target_kind = t.contiguous(), _lib.TARGET_LABELS_I64
    else:
        if target.numel() != b * c * n:
            raise AssertionError(
                f"ground truth has different shape ({tuple(target.shape)}) from input "
                f"({tuple(input.shape)})"
            )
        t = target.reshape(b, c, n)
        if code == _lib.F64:
            pl.target, pl.target_kind = t.double().contiguous(), _lib.TARGET_ONEHOT_F64
        else:
            pl.target, pl.target_kind = t.float().contiguous(), _lib.TARGET_ONEHOT_F32
    pl.btab, pl.rtab = bin_tables(pl.K, pl.soft, x.device)
    return pl


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device) -> int:
    """The current stream of ``dev`` as a raw handle (the accessor Triton
    uses; ``torch.cuda.current_stream`` builds a Python object first)."""
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def _d_values(pl: Plan) -> int:
    """Values of the forward's d: soft float32 outputs hold d rounded to
    float32 and its remainder ([2, B, C', K], the backward adds both);
    otherwise [B, C', K]."""
    bck = pl.B * pl.CL * pl.K
    return 2 * bck if pl.soft and pl.dtype_code != _lib.F64 else bck


def _d_shape(pl: Plan) -> Tuple[int, ...]:
    per = (pl.B, pl.CL, pl.K)
    return (2, *per) if _d_values(pl) > pl.B * pl.CL * pl.K else per


def saved_layout(pl: Plan, reduced: bool) -> Tuple[int, int, int, int]:
    """(values, d's byte offset, jac's, the per-class errors') of the one
    float32 allocation of a C++ loss call: coef, d, jac, then the per-class
    errors unless they are the returned loss."""
    bck, bc, nd = pl.B * pl.CL * pl.K, pl.B * pl.CL, _d_values(pl)
    return bck + nd + bc + (bc if reduced else 0), 4 * bck, 4 * (bck + nd), 4 * (bck + nd + bc)


@lru_cache(maxsize=256)
def _workspace_bytes(dims: Tuple[int, ...]) -> int:
    return _lib.lib().ace_workspace_bytes(*dims)


def hip_forward(pl: Plan, config: ACEConfig, stats: bool = False, shared: bool = True):
    """(loss, coef, d, jac, per_class, stats-or-None) via ``ace_forward``.
    d is [B, C', K], or for soft binning in float32 [2, B, C', K]: d rounded
    to float32 (``d[0]``) and its remainder (``d[1]``).
    ``shared``: coef, d and jac are views of one allocation (one allocator
    call instead of three); the custom op, whose outputs may not alias,
    passes False."""
    lib = _lib.lib()
    dev = pl.x.device
    stream = _stream(dev)
    binning = _lib.SOFT if pl.soft else _lib.HARD
    dims = (pl.B, pl.C, pl.N, pl.K, binning, pl.dtype_code, int(pl.include_bg), pl.target_kind)
    ws = workspace(dev, stream, _workspace_bytes(dims))
    f64 = pl.dtype_code == _lib.F64
    out_dtype = torch.float64 if f64 else torch.float32  # the outputs' type
    # coef, d and jac (all saved for backward) share one allocation; the
    # per-class errors and the loss, which the caller may receive and modify
    # in place, have their own
    bck, bc, nd = pl.B * pl.CL * pl.K, pl.B * pl.CL, _d_values(pl)
    if shared:
        saved = torch.empty(bck + nd + bc, dtype=out_dtype, device=dev)
        coef = saved[:bck].view(pl.B, pl.CL, pl.K)
        d = saved[bck:bck + nd].view(_d_shape(pl))
        jac = saved[bck + nd:].view(pl.B, pl.CL)
    else:
        coef = torch.empty((pl.B, pl.CL, pl.K), dtype=out_dtype, device=dev)
        d = torch.empty(_d_shape(pl), dtype=out_dtype, device=dev)
        jac = torch.empty((pl.B, pl.CL), dtype=out_dtype, device=dev)
    per_class = torch.empty((pl.B, pl.CL), dtype=out_dtype, device=dev)
    reduction = _REDUCTIONS[config.reduction]
    loss = torch.empty((), dtype=out_dtype, device=dev) if reduction != _lib.RED_NONE else None
    st = torch.empty((3, pl.B, pl.CL, pl.K), dtype=torch.float64, device=dev) if stats else None
    weights = class_weights(config, pl.CL)
    cw = class_weight_tensor(tuple(weights), dev, out_dtype) if weights is not None else None
    if f64:
        rc = lib.ace_forward_f64(
            pl.x.data_ptr(), pl.target.data_ptr(), pl.target_kind,
            pl.B, pl.C, pl.N, pl.K, binning, pl.act,
            int(pl.include_bg), int(config.ignore_empty_classes), reduction, int(pl.right),
            float(config.empty_weight), _ptr(cw), pl.btab.data_ptr(), _ptr(pl.rtab),
            ws.data_ptr(), ws.numel(),
            coef.data_ptr(), d.data_ptr(), jac.data_ptr(), per_class.data_ptr(), _ptr(loss),
            _ptr(st), stream,
        )
        _lib.check(rc, "ace_forward_f64")
    else:
        rc = lib.ace_forward(
            pl.x.data_ptr(), pl.dtype_code, pl.target.data_ptr(), pl.target_kind,
            pl.B, pl.C, pl.N, pl.K, binning, pl.act,
            int(pl.include_bg), int(config.ignore_empty_classes), reduction, int(pl.right),
            float(config.empty_weight), _ptr(cw), pl.btab.data_ptr(), _ptr(pl.rtab),
            ws.data_ptr(), ws.numel(),
            coef.data_ptr(), d.data_ptr(), jac.data_ptr(), per_class.data_ptr(), _ptr(loss),
            _ptr(st), stream,
        )
        _lib.check(rc, "ace_forward")
    if loss is None:
        loss = per_class.view(pl.B, pl.CL, *([1] * pl.spatial_ndim))
    return loss, coef, d, jac, per_class, st


def hip_backward(pl: Plan, coef: torch.Tensor, d: torch.Tensor, jac: torch.Tensor,
                 grad_output: torch.Tensor) -> torch.Tensor:
    """d loss / d input (input's shape and dtype) via ``ace_backward``."""
    lib = _lib.lib()
    dev = pl.x.device
    stream = _stream(dev)
    per_class = grad_output.dim() > 0
    go = grad_output
    f64 = pl.dtype_code == _lib.F64
    go_dtype = torch.float64 if f64 else torch.float32
    if go.dtype != go_dtype:
        go = go.to(go_dtype)
    go = go.reshape(-1) if per_class else go.reshape(())
    if not go.is_contiguous():
        go = go.contiguous()
    dx = torch.empty_like(pl.x)
    if pl.soft and not f64 and d.dim() == 3:
        # a float32 d without its remainder (not this forward's output)
        d = torch.cat([d.reshape(-1).float(), d.new_zeros(d.numel(), dtype=torch.float32)])
    if d.numel() != _d_values(pl) or not d.is_contiguous():
        raise ValueError(f"d must be the forward's contiguous {_d_shape(pl)} output, got {tuple(d.shape)}")
    if f64:
        rc = lib.ace_backward_f64(
            pl.x.data_ptr(), pl.target.data_ptr() if pl.soft else None, pl.target_kind,
            pl.B, pl.C, pl.N, pl.K, _lib.SOFT if pl.soft else _lib.HARD, pl.act,
            int(pl.include_bg), int(pl.right),
            pl.btab.data_ptr(), _ptr(pl.rtab),
            coef.data_ptr(), d.data_ptr(), jac.data_ptr(),
            go.data_ptr(), int(per_class),
            dx.data_ptr(), stream,
        )
        _lib.check(rc, "ace_backward_f64")
        return dx.view(pl.in_shape)
    rc = lib.ace_backward(
        pl.x.data_ptr(), pl.dtype_code,
        pl.target.data_ptr() if pl.soft else None, pl.target_kind,
        pl.B, pl.C, pl.N, pl.K, _lib.SOFT if pl.soft else _lib.HARD, pl.act,
        int(pl.include_bg), int(pl.right),
        pl.btab.data_ptr(), _ptr(pl.rtab),
        coef.data_ptr(), d.data_ptr(), jac.data_ptr(),
        go.data_ptr(), int(per_class),
        dx.data_ptr(), stream,
    )
    _lib.check(rc, "ace_backward")
    return dx.view(pl.in_shape)


class _Call:
    """A call signature -- (configuration, input shape and dtype, target
    shape and dtype, devices, stream) -- whose arguments of ``ace_forward`` /
    ``ace_backward`` are fixed, held by the C++ loss call
    (``_ace_autograd.Signature``): a call of that signature allocates its
    outputs, launches the forward and records the backward node in C++
    (``csrc/ace_autograd.cpp``), with no Python autograd Function.

    A signature qualifies when its kernel views are the caller's own tensors
    (contiguous, no dtype conversion) and the input is not float64 (its own
    entry points); it is remembered after its first call has succeeded.
    coef, d and jac (and the per-class errors, unless they are the returned
    loss) share one float32 allocation; the loss has its own (the caller may
    modify it in place).  The workspace is the stream's when the signature
    is made: a buffer that a larger problem later replaces is retired, never
    freed, and stays zero between calls on its stream."""

    __slots__ = ("sig", "ws", "tables")


def _build_call(pl: Plan, config: ACEConfig, stream: int) -> Optional[_Call]:
    if pl.dtype_code == _lib.F64:
        return None
    dev = pl.x.device
    binning = _lib.SOFT if pl.soft else _lib.HARD
    dims = (pl.B, pl.C, pl.N, pl.K, binning, pl.dtype_code, int(pl.include_bg), pl.target_kind)
    ws = workspace(dev, stream, _workspace_bytes(dims))
    weights = class_weights(config, pl.CL)
    cw = class_weight_tensor(tuple(weights), dev) if weights is not None else None
    reduction = _REDUCTIONS[config.reduction]
    reduced = reduction != _lib.RED_NONE
    c = _Call()
    c.sig = _lib.autograd().make_signature(
        pl.dtype_code, pl.target_kind, pl.B, pl.C, pl.N, pl.K, binning, pl.act, int(pl.include_bg),
        int(config.ignore_empty_classes), reduction, int(pl.right), float(config.empty_weight),
        _ptr(cw) or 0, pl.btab.data_ptr(), _ptr(pl.rtab) or 0, ws.data_ptr(), ws.numel(),
        *saved_layout(pl, reduced), reduced, pl.soft,
        [] if reduced else [pl.B, pl.CL, *([1] * pl.spatial_ndim)])
    c.ws, c.tables = ws, (cw, pl.btab, pl.rtab)  # kept alive with the signature
    return c


# signature -> _Call (None: the general path); bounded, cleared when full
_CALLS: Dict[Tuple[Any, ...], Optional[_Call]] = {}
_MAX_CALLS = 256


class _HipACELoss(torch.autograd.Function):
    """The general path: calls that no remembered signature covers."""

    @staticmethod
    def forward(ctx: Any, input: torch.Tensor, target: torch.Tensor, config: ACEConfig,
                pl: Plan) -> torch.Tensor:
        loss, coef, d, jac, _, _ = hip_forward(pl, config)
        # the kernel views of input / target (same storage and version counter
        # as the caller's tensors) go through save_for_backward
        ctx.save_for_backward(pl.x.detach(), pl.target.detach(), coef, d, jac)
        pl.x = pl.target = None
        ctx.plan = pl
        return loss

    @staticmethod
    def backward(ctx: Any, grad_output: torch.Tensor) -> Tuple[Optional[torch.Tensor], None, None, None]:
        x, target, coef, d, jac = ctx.saved_tensors
        pl = ctx.plan
        pl.x, pl.target = x, target
        try:
            dx = hip_backward(pl, coef, d, jac, grad_output)
        finally:
            pl.x = pl.target = None
        return dx, None, None, None


def hip_ace(input: torch.Tensor, target: torch.Tensor, config: ACEConfig) -> torch.Tensor:
    """Registry entry ``fn(input, target, config) -> loss``.

    A remembered signature runs in C++ (``_Call``); any other call builds a
    ``Plan`` and runs the autograd Function above (or, with no gradient to
    record, the forward alone), and remembers its signature once it has
    succeeded.  The target gets no gradient (None), as in the reference's
    ``_V6Loss.backward`` (``impls/v6_triton.py:107-111``)."""
    stream = _stream(input.device) if input.is_cuda else 0
    key = (config, input.shape, input.dtype, target.shape, target.dtype, input.get_device(),
           target.get_device(), stream)
    call = _CALLS.get(key)
    # a target that needs a gradient (and gets none, as in the reference's
    # autograd Function) takes the Function below, so that the loss records
    # autograd history even when the input needs no gradient
    if call is not None and not target.requires_grad and input.is_contiguous() and target.is_contiguous():
        loss: torch.Tensor = _lib.autograd().ace_loss(input, target, call.sig)
        return loss
    pl = make_plan(input, target, config)
    own = (pl.x.data_ptr() == input.data_ptr() and pl.x.dtype == input.dtype and input.is_contiguous()
           and pl.target.data_ptr() == target.data_ptr() and pl.target.dtype == target.dtype
           and target.is_contiguous())
    if torch.is_grad_enabled() and (input.requires_grad or target.requires_grad):
        loss = _HipACELoss.apply(input, target, config, pl)
    else:
        loss = hip_forward(pl, config)[0]
    if key not in _CALLS and not capturing(input.device):
        if len(_CALLS) >= _MAX_CALLS:
            _CALLS.clear()
        pl.x, pl.target = input, target  # for _build_call: device, tables (kernel views not needed)
        _CALLS[key] = _build_call(pl, config, stream) if own else None
    return loss


register(
    "hip_mi355x",
    description="MI355X HIP kernels: fused softmax/binning/histogram forward, one-pass backward",
    devices=frozenset({"cuda"}),
)(hip_ace)


# ---------------------------------------------------------------- custom ops
# The same kernels as ``torch.library`` custom ops with fake (meta) kernels
# and an autograd formula, so that ``torch.compile(fullgraph=True)`` of a
# network plus this loss traces through it without graph breaks -- the
# packaging of the reference's ``v6_forward`` / ``v6_backward``
# (``src/ace_kernels/impls/v6_triton.py:141-216``).  The config travels as its
# JSON text, a compile-time constant.

Outputs = Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]


@lru_cache(maxsize=64)
def _config(config_json: str) -> ACEConfig:
    return ACEConfig.model_validate_json(config_json)


def _dump(config: ACEConfig) -> str:
    return config.model_dump_json()


# constant for torch.compile (pydantic models are not traceable): a compiled
# function must not swap configs between calls
config_arg = torch.compiler.assume_constant_result(_dump)


@torch.library.custom_op("ace_kernels::hip_forward", mutates_args=())
def hip_forward_op(input: torch.Tensor, target: torch.Tensor, config_json: str) -> Outputs:
    """mL1-ACE forward: (loss, coef, d, jac) from one ``ace_forward`` launch."""
    config = _config(config_json)
    loss, coef, d, jac, _, _ = hip_forward(make_plan(input, target, config), config, shared=False)
    # a custom op may not return a view of an internal buffer: copy the "none" view
    return (loss.clone() if loss.dim() else loss), coef, d, jac


@hip_forward_op.register_fake
def _(input: torch.Tensor, target: torch.Tensor, config_json: str) -> Outputs:
    config = _config(config_json)
    b, c = input.shape[:2]
    cl = c - (1 if (not config.include_background and c > 1) else 0)
    out = torch.float64 if input.dtype == torch.float64 else torch.float32
    per_bin = input.new_empty((b, cl, config.num_bins), dtype=out)
    loss_shape = (b, cl, *([1] * (input.dim() - 2))) if config.reduction == "none" else ()
    loss = input.new_empty(loss_shape, dtype=out)
    jac = input.new_empty((b, cl), dtype=out)
    # soft float32: d and its remainder
    d_shape = (2, b, cl, config.num_bins) if config.binning == "soft" and out == torch.float32 else per_bin.shape
    return loss, per_bin, input.new_empty(d_shape, dtype=out), jac


@torch.library.custom_op("ace_kernels::hip_backward", mutates_args=())
def hip_backward_op(input: torch.Tensor, target: torch.Tensor, coef: torch.Tensor,
                    d: torch.Tensor, jac: torch.Tensor, grad_output: torch.Tensor,
                    config_json: str) -> torch.Tensor:
    """d loss / d input from one ``ace_backward`` launch."""
    return hip_backward(make_plan(input, target, _config(config_json)), coef, d, jac, grad_output)


@hip_backward_op.register_fake
def _(input: torch.Tensor, target: torch.Tensor, coef: torch.Tensor, d: torch.Tensor,
      jac: torch.Tensor, grad_output: torch.Tensor, config_json: str) -> torch.Tensor:
    return torch.empty_like(input)


def _setup_context(ctx: Any, inputs: Tuple[Any, ...], output: Outputs) -> None:
    input, target, config_json = inputs
    _, coef, d, jac = output
    ctx.config_json = config_json
    ctx.set_materialize_grads(False)  # coef / d / jac get no gradient: no zero fills
    ctx.save_for_backward(input, target, coef, d, jac)


def _op_backward(ctx: Any, grad_loss: torch.Tensor, *_unused: torch.Tensor):
    input, target, coef, d, jac = ctx.saved_tensors
    dx = hip_backward_op(input, target, coef, d, jac, grad_loss, ctx.config_json)
    return dx, None, None


hip_forward_op.register_autograd(_op_backward, setup_context=_setup_context)


def hip_ace_op(input: torch.Tensor, target: torch.Tensor, config: ACEConfig) -> torch.Tensor:
    """Registry entry over the custom ops (compile-friendly)."""
    loss: torch.Tensor = hip_forward_op(input, target, config_arg(config))[0]
    return loss


def hip_ace_op_json(input: torch.Tensor, target: torch.Tensor, config_json: str) -> torch.Tensor:
    """The custom ops with the config already as JSON text: what the drop-in
    modules call under ``torch.compile`` (a string attribute is a trace-time
    constant; this torch version cannot fold the pydantic config itself)."""
    loss: torch.Tensor = hip_forward_op(input, target, config_json)[0]
    return loss


register(
    "hip_mi355x_op",
    description="hip_mi355x as torch.library custom ops (torch.compile without graph breaks)",
    devices=frozenset({"cuda"}),
)(hip_ace_op)
