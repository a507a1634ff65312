"""``jit_thc::*`` operators of the non-shared (triangular lazy / v2) LTHC interface.

With a separate read R_l = alpha_l and write P_l = beta_l per layer, the
workspace input of layer l is (local_thc.py:1434-1451)

    z_l = R_l(x0) + sum_{j<l} gamma[l, j] * dz_j,   gamma[l, j, c] = sum_k alpha_l[c,k] beta_j[c,k]

and the final high-resolution state is the usual materialisation.  The
reference computes the 12 bases R_l(x0) with ``all_base_b4_12[_split]`` and
the sums with ``triangular_accumulate*`` (local_thc_triton_kernels.py:684-1012,
1922-2670).  This module registers the same names, schemas and autograd
formulas on the gfx950 HIP library:

* the bases are the multi-weight read (``lthc_read_multi_fwd``), their
  gradient the sum of writes (``lthc_materialise_fwd`` without a base) and the
  read-weight gradient ``lthc_weight_grad``;
* the triangular sums are ``lthc_ws_accumulate_fwd`` / ``_bwd``.

The reference's ops are fixed to the 64x64 / 16x16 geometry and 12 layers;
these accept any square grid of cell side 4, and the stacked forms any depth up
to 24 (MAX_WS_DEPTH).  Weight gradients are reduced in a fixed order (the reference uses fp32
atomics).  As in the reference, gradients of gamma are computed in fp32 and
cast to gamma's dtype.
"""

from __future__ import annotations

from typing import Sequence

import torch
from torch import Tensor

from . import _abi
from .ops import (
    K,
    S,
    _check_weight,
    _fake,
    _hi_geom,
    _launch_materialise,
    _launch_read_multi,
    _launch_weight_grad,
    _lo_geom,
    _on_device,
    _on_gpu,
    _prep,
    _prep_w,
    _same_dtype,
)

MAX_WS_DEPTH = 24


# ---------------------------------------------------------------------------
# launches
# ---------------------------------------------------------------------------
def _check_ws(base: Tensor, dzs: Sequence[Tensor], gamma: Tensor) -> tuple[int, int]:
    if base.dim() != 3:
        raise ValueError(f"base must be [B,M,C], got {tuple(base.shape)}")
    c = base.shape[2]
    L = len(dzs)
    if not 1 <= L <= MAX_WS_DEPTH:
        raise ValueError(f"depth {L} outside 1..{MAX_WS_DEPTH}")
    for i, dz in enumerate(dzs):
        if dz.shape != base.shape:
            raise ValueError(f"dz{i} shape {tuple(dz.shape)} does not match base {tuple(base.shape)}")
    if gamma.dim() != 2 or gamma.shape[0] < L or gamma.shape[1] != c:
        raise ValueError(f"gamma must be [>= {L}, {c}], got {tuple(gamma.shape)}")
    if c % 4 != 0:
        raise ValueError(f"channels {c} must be a multiple of 4")
    _abi.code(gamma)
    return base.numel() // c, c


def _ws_forward(base: Tensor, dzs: Sequence[Tensor], gamma: Tensor) -> Tensor:
    """out = base + sum_{i<L} gamma[i] * dzs[i] (L = len(dzs); gamma rows beyond L are unused)."""
    _on_gpu(base, *dzs, gamma)
    rows, c = _check_ws(base, dzs, gamma)
    base = _prep(base)
    dzs = _same_dtype(base, [_prep(d) for d in dzs])
    gamma = gamma.contiguous()
    out = torch.empty_like(base)
    with _on_device(base):
        rc = _abi.load().lthc_ws_accumulate_fwd(
            base.data_ptr(), _abi.ptr_array(dzs), _abi.code(base), gamma.data_ptr(), _abi.code(gamma),
            out.data_ptr(), rows, c, len(dzs), _abi.stream_of(base),
        )  # fmt: skip
    _abi.check(rc, "lthc_ws_accumulate_fwd")
    return out


def _ws_backward(grad: Tensor, dzs: Sequence[Tensor] | None, gamma: Tensor, L: int, want_dz: bool):
    """(list of gamma[i] * grad for i < L or None, fp32 [L, C] sum_r grad * dzs[i] or None)."""
    _on_gpu(grad, gamma)
    c = grad.shape[-1]
    rows = grad.numel() // c
    grad = _prep(grad)
    gamma = gamma.contiguous()
    gdz = [torch.empty_like(grad) for _ in range(L)] if want_dz else None
    gg = ws = None
    if dzs is not None:
        dzs = _same_dtype(grad, [_prep(d) for d in dzs[:L]])
        gg = torch.empty((L, c), device=grad.device, dtype=torch.float32)
        ws = torch.empty((max(_abi.ws_accumulate_bwd_workspace_bytes(rows, c, L), 16),), device=grad.device, dtype=torch.uint8)
    with _on_device(grad):
        rc = _abi.load().lthc_ws_accumulate_bwd(
            grad.data_ptr(), _abi.ptr_array(dzs) if dzs is not None else None, _abi.code(grad), gamma.data_ptr(),
            _abi.code(gamma), _abi.ptr_array(gdz) if gdz is not None else None, _abi.ptr(gg), rows, c, L,
            _abi.ptr(ws), 0 if ws is None else ws.numel(), _abi.stream_of(grad),
        )  # fmt: skip
    _abi.check(rc, "lthc_ws_accumulate_bwd")
    return gdz, gg


@torch.library.custom_op("jit_thc::ws_accumulate_backward", mutates_args=())
def ws_accumulate_backward(grad: Tensor, dzs: list[Tensor], gamma: Tensor, L: int, want_dz: bool) -> tuple[list[Tensor], Tensor]:
    """_ws_backward as an op (the triangular ops' autograd backwards call it, so torch.compile traces them as one
    opaque node): ([gamma[i] * grad for i < L] or [] without want_dz, fp32 [L, C] sum grad * dzs[i] or an empty
    tensor when dzs is empty)."""
    gdz, gg = _ws_backward(grad, dzs if dzs else None, gamma, L, want_dz)
    return (gdz if gdz is not None else []), (gg if gg is not None else grad.new_empty((0,), dtype=torch.float32))


@_fake(ws_accumulate_backward)
def _(grad: Tensor, dzs: list[Tensor], gamma: Tensor, L: int, want_dz: bool):
    gdz = [torch.empty_like(grad) for _ in range(L)] if want_dz else []
    gg = grad.new_empty((L, grad.shape[-1]) if dzs else (0,), dtype=torch.float32)
    return gdz, gg


def _ws_backward_op(grad: Tensor, dzs: Sequence[Tensor] | None, gamma: Tensor, L: int, want_dz):
    """_ws_backward's (gdz list or None, gg or None) through the op.  `want_dz` is a bool, or the per-layer flags
    of needs_input_grad for a list argument (any of them)."""
    want_dz = any(want_dz) if isinstance(want_dz, (list, tuple)) else bool(want_dz)
    gdz, gg = ws_accumulate_backward(grad, list(dzs) if dzs is not None else [], gamma, L, want_dz)
    return (gdz if want_dz else None), (gg if dzs is not None else None)


# ---------------------------------------------------------------------------
# jit_thc::triangular_accumulate_traceable (stacked, any depth; :1922-2012)
# ---------------------------------------------------------------------------
@torch.library.custom_op("jit_thc::triangular_accumulate_traceable", mutates_args=())
def triangular_accumulate_traceable(base: Tensor, dz_stack: Tensor, gamma: Tensor) -> Tensor:
    """base + sum_l gamma[l][c] * dz_stack[l] for base [B,M,C], dz_stack [L,B,M,C], gamma [L,C]."""
    if dz_stack.dim() != 4:
        raise ValueError(f"dz_stack must be [L,B,M,C], got {tuple(dz_stack.shape)}")
    return _ws_forward(base, list(dz_stack.unbind(0)), gamma)


@_fake(triangular_accumulate_traceable)
def _(base: Tensor, dz_stack: Tensor, gamma: Tensor) -> Tensor:
    return torch.empty_like(base)


@torch.library.custom_op("jit_thc::triangular_accumulate_grad_dz", mutates_args=())
def triangular_accumulate_grad_dz_traceable(grad_out: Tensor, gamma: Tensor) -> Tensor:
    """[L,B,M,C] of gamma[l][c] * grad_out in grad_out.dtype."""
    L = gamma.shape[0]
    gdz, _ = _ws_backward(grad_out, None, gamma, L, True)
    return torch.stack(gdz)


@_fake(triangular_accumulate_grad_dz_traceable)
def _(grad_out: Tensor, gamma: Tensor) -> Tensor:
    return grad_out.new_empty((gamma.shape[0], *grad_out.shape))


@torch.library.custom_op("jit_thc::triangular_accumulate_grad_gamma", mutates_args=())
def triangular_accumulate_grad_gamma_traceable(grad_out: Tensor, dz_stack: Tensor, gamma: Tensor) -> Tensor:
    """fp32 [L,C] of sum_{b,m} grad_out * dz_stack[l] (fixed summation order)."""
    _, gg = _ws_backward(grad_out, list(dz_stack.unbind(0)), gamma, gamma.shape[0], False)
    return gg


@_fake(triangular_accumulate_grad_gamma_traceable)
def _(grad_out: Tensor, dz_stack: Tensor, gamma: Tensor) -> Tensor:
    return grad_out.new_empty((gamma.shape[0], grad_out.shape[-1]), dtype=torch.float32)


def _setup_tri_ctx(ctx, inputs, output):
    _, dz_stack, gamma = inputs
    ctx.save_for_backward(dz_stack, gamma)


def _backward_tri(ctx, grad_out):
    # local_thc_triton_kernels.py:1996-2004: grad_base is grad_out itself.
    dz_stack, gamma = ctx.saved_tensors
    grad_out = grad_out.contiguous()
    need = ctx.needs_input_grad
    gdz, gg = _ws_backward_op(grad_out, list(dz_stack.unbind(0)) if need[2] else None, gamma, gamma.shape[0], need[1])
    return (
        grad_out,
        torch.stack(gdz) if gdz is not None else None,
        gg.to(gamma.dtype) if gg is not None else None,
    )


torch.library.register_autograd(triangular_accumulate_traceable, _backward_tri, setup_context=_setup_tri_ctx)


# ---------------------------------------------------------------------------
# jit_thc::triangular_accumulate_list: the same sum with the layers as a list
# (no dz stack copy; any depth 1..24, gamma rows beyond len(dzs) unused)
# ---------------------------------------------------------------------------
@torch.library.custom_op("jit_thc::triangular_accumulate_list", mutates_args=())
def triangular_accumulate_list(base: Tensor, dzs: list[Tensor], gamma: Tensor) -> Tensor:
    """base + sum_{i < len(dzs)} gamma[i][c] * dzs[i] for base [B,M,C], gamma [>= len(dzs), C]."""
    return _ws_forward(base, dzs, gamma)


@_fake(triangular_accumulate_list)
def _(base: Tensor, dzs: list[Tensor], gamma: Tensor) -> Tensor:
    return torch.empty_like(base)


def _setup_tri_list_ctx(ctx, inputs, output):
    _, dzs, gamma = inputs
    ctx.save_for_backward(*dzs, gamma)
    ctx.L = len(dzs)


def _backward_tri_list(ctx, grad_out):
    saved = ctx.saved_tensors
    dzs, gamma = list(saved[: ctx.L]), saved[ctx.L]
    grad_out = grad_out.contiguous()
    need = ctx.needs_input_grad
    gdz, gg = _ws_backward_op(grad_out, dzs if need[2] else None, gamma, ctx.L, need[1])
    grad_gamma = None
    if gg is not None:
        if gamma.shape[0] > ctx.L:
            full = torch.zeros(gamma.shape, device=gg.device, dtype=torch.float32)
            full[: ctx.L] = gg
            gg = full
        grad_gamma = gg.to(gamma.dtype)
    return grad_out, gdz, grad_gamma


torch.library.register_autograd(triangular_accumulate_list, _backward_tri_list, setup_context=_setup_tri_list_ctx)


# ---------------------------------------------------------------------------
# 12 separate layers (:2015-2157) and the active-prefix forms (:2161-2488)
# ---------------------------------------------------------------------------
_DZ12 = ", ".join(f"Tensor dz{i}" for i in range(12))


def _tri12_forward(base: Tensor, dzs: Sequence[Tensor], gamma: Tensor, active: int) -> Tensor:
    if base.dim() != 3 or gamma.dim() != 2 or tuple(gamma.shape) != (12, base.shape[2]):
        raise ValueError(
            f"triangular_accumulate_b4_12 expects base [B,M,C] and gamma [12,C], got {tuple(base.shape)} and {tuple(gamma.shape)}"
        )
    for i, dz in enumerate(dzs):
        if dz.shape != base.shape:
            raise ValueError(f"triangular_accumulate_b4_12 dz{i} shape {tuple(dz.shape)} does not match base {tuple(base.shape)}")
    return _ws_forward(base, list(dzs[:active]), gamma)


def _tri12_grad_dz(grad_out: Tensor, gamma: Tensor, active: int) -> Tensor:
    gdz, _ = _ws_backward(grad_out, None, gamma, active, True)
    return torch.stack(gdz)


def _tri12_grad_gamma(grad_out: Tensor, dzs: Sequence[Tensor], gamma: Tensor, active: int) -> Tensor:
    _, gg = _ws_backward(grad_out, list(dzs), gamma, active, False)
    if active == 12:
        return gg
    full = torch.zeros((12, grad_out.shape[-1]), device=grad_out.device, dtype=torch.float32)
    full[:active] = gg
    return full


torch.library.define(
    "jit_thc::triangular_accumulate_b4_12_ptr_traceable", f"(Tensor base, {_DZ12}, Tensor gamma) -> Tensor"
)
torch.library.define("jit_thc::triangular_accumulate_b4_12_ptr_grad_dz", "(Tensor grad_out, Tensor gamma) -> Tensor")
torch.library.define(
    "jit_thc::triangular_accumulate_b4_12_ptr_grad_gamma", f"(Tensor grad_out, {_DZ12}, Tensor gamma) -> Tensor"
)
torch.library.define(
    "jit_thc::triangular_accumulate_b4_12_ptr_active", f"(Tensor base, {_DZ12}, Tensor gamma, int active) -> Tensor"
)
torch.library.define(
    "jit_thc::triangular_accumulate_b4_12_ptr_active_grad_dz", "(Tensor grad_out, Tensor gamma, int active) -> Tensor"
)
torch.library.define(
    "jit_thc::triangular_accumulate_b4_12_ptr_active_grad_gamma",
    f"(Tensor grad_out, {_DZ12}, Tensor gamma, int active) -> Tensor",
)


def _check_active(active: int) -> int:
    if not 1 <= active <= 11:
        raise ValueError(f"active must be in [1, 11], got {active}")
    return int(active)


@torch.library.impl("jit_thc::triangular_accumulate_b4_12_ptr_traceable", "CUDA")
def _tri12_impl(base, *args):
    return _tri12_forward(base, args[:12], args[12], 12)


@torch.library.impl("jit_thc::triangular_accumulate_b4_12_ptr_grad_dz", "CUDA")
def _tri12_grad_dz_impl(grad_out, gamma):
    return _tri12_grad_dz(grad_out, gamma, 12)


@torch.library.impl("jit_thc::triangular_accumulate_b4_12_ptr_grad_gamma", "CUDA")
def _tri12_grad_gamma_impl(grad_out, *args):
    return _tri12_grad_gamma(grad_out, args[:12], args[12], 12)


@torch.library.impl("jit_thc::triangular_accumulate_b4_12_ptr_active", "CUDA")
def _tri12a_impl(base, *args):
    return _tri12_forward(base, args[:12], args[12], _check_active(args[13]))


@torch.library.impl("jit_thc::triangular_accumulate_b4_12_ptr_active_grad_dz", "CUDA")
def _tri12a_grad_dz_impl(grad_out, gamma, active):
    return _tri12_grad_dz(grad_out, gamma, _check_active(active))


@torch.library.impl("jit_thc::triangular_accumulate_b4_12_ptr_active_grad_gamma", "CUDA")
def _tri12a_grad_gamma_impl(grad_out, *args):
    return _tri12_grad_gamma(grad_out, args[:12], args[12], _check_active(args[13]))


def _cpu_refusal(name):
    def refuse(*args):
        raise ValueError(f"LTHC HIP ops need GPU tensors (there is no CPU fallback): {name}")

    return refuse


for _name in (
    "triangular_accumulate_b4_12_ptr_traceable",
    "triangular_accumulate_b4_12_ptr_grad_dz",
    "triangular_accumulate_b4_12_ptr_grad_gamma",
    "triangular_accumulate_b4_12_ptr_active",
    "triangular_accumulate_b4_12_ptr_active_grad_dz",
    "triangular_accumulate_b4_12_ptr_active_grad_gamma",
):
    torch.library.impl(f"jit_thc::{_name}", "CPU")(_cpu_refusal(_name))


@_fake("jit_thc::triangular_accumulate_b4_12_ptr_traceable")
def _(base, *args):
    return torch.empty_like(base)


@_fake("jit_thc::triangular_accumulate_b4_12_ptr_grad_dz")
def _(grad_out, gamma):
    return grad_out.new_empty((12, *grad_out.shape))


@_fake("jit_thc::triangular_accumulate_b4_12_ptr_grad_gamma")
def _(grad_out, *args):
    return grad_out.new_empty((12, grad_out.shape[-1]), dtype=torch.float32)


@_fake("jit_thc::triangular_accumulate_b4_12_ptr_active")
def _(base, *args):
    return torch.empty_like(base)


@_fake("jit_thc::triangular_accumulate_b4_12_ptr_active_grad_dz")
def _(grad_out, gamma, active):
    return grad_out.new_empty((active, *grad_out.shape))


@_fake("jit_thc::triangular_accumulate_b4_12_ptr_active_grad_gamma")
def _(grad_out, *args):
    return grad_out.new_empty((12, grad_out.shape[-1]), dtype=torch.float32)


def _setup_tri12_ctx(ctx, inputs, output):
    ctx.save_for_backward(*inputs[1:14])
    ctx.active = int(inputs[14]) if len(inputs) > 14 else 12


def _tri12_grads(ctx, grad_out) -> tuple:
    """Gradients of (base, dz0..dz11, gamma).  local_thc_triton_kernels.py:2141-2151 and :2470-2482:
    grad_base is grad_out itself; the layers beyond the active prefix get no gradient."""
    saved = ctx.saved_tensors
    dzs, gamma, active = saved[:12], saved[12], ctx.active
    grad_out = grad_out.contiguous()
    need = ctx.needs_input_grad
    want_dz = any(need[1 : 1 + active])
    gdz, gg = _ws_backward_op(grad_out, list(dzs[:active]) if need[13] else None, gamma, active, want_dz)
    grad_dzs = (tuple(gdz) if gdz is not None else (None,) * active) + (None,) * (12 - active)
    grad_gamma = None
    if gg is not None:
        if active < 12:
            full = torch.zeros((12, gamma.shape[1]), device=gg.device, dtype=torch.float32)
            full[:active] = gg
            gg = full
        grad_gamma = gg.to(gamma.dtype)
    return (grad_out, *grad_dzs, grad_gamma)


def _backward_tri12(ctx, grad_out):
    return _tri12_grads(ctx, grad_out)


def _backward_tri12_active(ctx, grad_out):
    return _tri12_grads(ctx, grad_out) + (None,)  # no gradient for the int `active`


torch.library.register_autograd(
    "jit_thc::triangular_accumulate_b4_12_ptr_traceable", _backward_tri12, setup_context=_setup_tri12_ctx
)
torch.library.register_autograd(
    "jit_thc::triangular_accumulate_b4_12_ptr_active", _backward_tri12_active, setup_context=_setup_tri12_ctx
)


def triangular_accumulate_b4_12_ptr_traceable(base, *args):
    return torch.ops.jit_thc.triangular_accumulate_b4_12_ptr_traceable(base, *args)


def triangular_accumulate_b4_12_ptr_active_traceable(base, *args):
    return torch.ops.jit_thc.triangular_accumulate_b4_12_ptr_active(base, *args)


def _make_active_op(active: int):
    """jit_thc::triangular_accumulate_b4_12_ptr_active{active}: the active-prefix op with the prefix fixed in
    the name (local_thc_triton_kernels.py:2161-2322)."""
    name = f"triangular_accumulate_b4_12_ptr_active{active}"
    torch.library.define(f"jit_thc::{name}", f"(Tensor base, {_DZ12}, Tensor gamma) -> Tensor")
    torch.library.define(f"jit_thc::{name}_grad_dz", "(Tensor grad_out, Tensor gamma) -> Tensor")
    torch.library.define(f"jit_thc::{name}_grad_gamma", f"(Tensor grad_out, {_DZ12}, Tensor gamma) -> Tensor")
    torch.library.impl(f"jit_thc::{name}", "CUDA")(lambda base, *a: _tri12_forward(base, a[:12], a[12], active))
    torch.library.impl(f"jit_thc::{name}_grad_dz", "CUDA")(lambda g, gamma: _tri12_grad_dz(g, gamma, active))
    torch.library.impl(f"jit_thc::{name}_grad_gamma", "CUDA")(lambda g, *a: _tri12_grad_gamma(g, a[:12], a[12], active))
    for suffix in ("", "_grad_dz", "_grad_gamma"):
        torch.library.impl(f"jit_thc::{name}{suffix}", "CPU")(_cpu_refusal(name + suffix))
    _fake(f"jit_thc::{name}")(lambda base, *a: torch.empty_like(base))
    _fake(f"jit_thc::{name}_grad_dz")(lambda g, gamma: g.new_empty((active, *g.shape)))
    _fake(f"jit_thc::{name}_grad_gamma")(
        lambda g, *a: g.new_empty((12, g.shape[-1]), dtype=torch.float32)
    )

    def setup(ctx, inputs, output):
        ctx.save_for_backward(*inputs[1:14])
        ctx.active = active

    def backward(ctx, grad_out):
        return _tri12_grads(ctx, grad_out)

    torch.library.register_autograd(f"jit_thc::{name}", backward, setup_context=setup)
    return getattr(torch.ops.jit_thc, name)


triangular_accumulate_b4_12_ptr_active_traceable_ops = tuple(_make_active_op(a) for a in range(1, 12))


# ---------------------------------------------------------------------------
# all_base_b4_12 / all_base_b4_12_split (:2489-2670): the per-layer bases R_l(x0)
# ---------------------------------------------------------------------------
def _check_alpha_stack(x0: Tensor, alpha_stack: Tensor) -> tuple[int, int, int, int]:
    b, g, c = _hi_geom(x0, "x0")
    # The gradient w.r.t. x0 is a base-less materialisation, which the library supports up to MAX_WS_DEPTH layers.
    if alpha_stack.dim() != 3 or tuple(alpha_stack.shape[1:]) != (c, K) or not 1 <= alpha_stack.shape[0] <= MAX_WS_DEPTH:
        raise ValueError(f"alpha_stack must be [L,{c},{K}] with 1 <= L <= {MAX_WS_DEPTH}, got {tuple(alpha_stack.shape)}")
    return b, g, c, alpha_stack.shape[0]


def _bases(x0: Tensor, alpha_stack: Tensor, stacked: bool) -> Tensor | list[Tensor]:
    """The L bases from one read_multi pass: written straight into one [L,B,M,C] tensor when stacked, else into
    L separate [B,M,C] tensors."""
    _on_gpu(x0, alpha_stack)
    b, g, c, L = _check_alpha_stack(x0, alpha_stack)
    x0 = _prep(x0)
    alphas = list(_prep_w(alpha_stack, x0.dtype).unbind(0))
    if stacked:
        out = torch.empty((L, b, g * g, c), device=x0.device, dtype=x0.dtype)
        _launch_read_multi(x0, alphas, list(out.unbind(0)))
        return out
    outs = [torch.empty((b, g * g, c), device=x0.device, dtype=x0.dtype) for _ in range(L)]
    _launch_read_multi(x0, alphas, outs)
    return outs


@torch.library.custom_op("jit_thc::all_base_b4_12_traceable", mutates_args=())
def all_base_b4_12_traceable(x0: Tensor, alpha_stack: Tensor) -> Tensor:
    """[L,B,M,C] of R_{alpha_l}(x0) for every l, one pass over x0."""
    return _bases(x0, alpha_stack, stacked=True)


@_fake(all_base_b4_12_traceable)
def _(x0: Tensor, alpha_stack: Tensor) -> Tensor:
    b, g, c = _hi_geom(x0, "x0")
    return x0.new_empty((alpha_stack.shape[0], b, g * g, c))


@torch.library.custom_op("jit_thc::all_base_b4_12_grad_x", mutates_args=())
def all_base_b4_12_grad_x_traceable(grad_base: Tensor, alpha_stack: Tensor) -> Tensor:
    """sum_l R_{alpha_l}^T(grad_base[l]) as [B,H,H,C] (one pass, no base tensor)."""
    _on_gpu(grad_base, alpha_stack)
    if grad_base.dim() != 4:
        raise ValueError(f"grad_base must be [L,B,M,C], got {tuple(grad_base.shape)}")
    L, b, m, c = grad_base.shape
    grads = [_prep(t) for t in grad_base.unbind(0)]
    _, g, _ = _lo_geom(grads[0], "grad_base")
    if tuple(alpha_stack.shape) != (L, c, K) or L > MAX_WS_DEPTH:
        raise ValueError(f"alpha_stack must be [{L},{c},{K}] with L <= {MAX_WS_DEPTH}, got {tuple(alpha_stack.shape)}")
    alphas = list(_prep_w(alpha_stack, grad_base.dtype).unbind(0))
    out = torch.empty((b, g * S, g * S, c), device=grad_base.device, dtype=grad_base.dtype)
    _launch_materialise(None, grads, alphas, out)
    return out


@_fake(all_base_b4_12_grad_x_traceable)
def _(grad_base: Tensor, alpha_stack: Tensor) -> Tensor:
    L, b, m, c = grad_base.shape
    h = int(round(m**0.5)) * S
    return grad_base.new_empty((b, h, h, c))


@torch.library.custom_op("jit_thc::all_base_b4_12_grad_alpha", mutates_args=())
def all_base_b4_12_grad_alpha_traceable(x0: Tensor, grad_base: Tensor, alpha_stack: Tensor) -> Tensor:
    """fp32 [L,C,16] of sum_{b,m} x0[b,m,k,c] grad_base[l][b,m,c] (fixed summation order)."""
    _on_gpu(x0, grad_base, alpha_stack)
    x0 = _prep(x0)
    lows = _same_dtype(x0, [_prep(t) for t in grad_base.unbind(0)])
    return _launch_weight_grad(x0, lows)


@_fake(all_base_b4_12_grad_alpha_traceable)
def _(x0: Tensor, grad_base: Tensor, alpha_stack: Tensor) -> Tensor:
    return x0.new_empty((grad_base.shape[0], x0.shape[3], K), dtype=torch.float32)


def _setup_all_base_ctx(ctx, inputs, output):
    x0, alpha_stack = inputs
    ctx.save_for_backward(x0, alpha_stack)


def _backward_all_base(ctx, grad_base):
    x0, alpha_stack = ctx.saved_tensors
    grad_base = grad_base.contiguous()
    need = ctx.needs_input_grad
    grad_x = all_base_b4_12_grad_x_traceable(grad_base, alpha_stack) if need[0] else None
    grad_alpha = all_base_b4_12_grad_alpha_traceable(x0, grad_base, alpha_stack).to(alpha_stack.dtype) if need[1] else None
    return grad_x, grad_alpha


torch.library.register_autograd(all_base_b4_12_traceable, _backward_all_base, setup_context=_setup_all_base_ctx)


@torch.library.custom_op("jit_thc::all_base_b4_12_split_traceable", mutates_args=())
def all_base_b4_12_split_traceable(x0: Tensor, alpha_stack: Tensor) -> list[Tensor]:
    """The L bases R_{alpha_l}(x0) as separate [B,M,C] tensors (one pass over x0)."""
    return _bases(x0, alpha_stack, stacked=False)


@_fake(all_base_b4_12_split_traceable)
def _(x0: Tensor, alpha_stack: Tensor) -> list[Tensor]:
    b, g, c = _hi_geom(x0, "x0")
    return [x0.new_empty((b, g * g, c)) for _ in range(alpha_stack.shape[0])]


@torch.library.custom_op("jit_thc::all_base_b4_12_split_grad_alpha", mutates_args=())
def all_base_b4_12_split_grad_alpha_traceable(x0: Tensor, grad_base: Tensor) -> Tensor:
    """fp32 [L,C,16] of sum_{b,m} x0[b,m,k,c] grad_base[l][b,m,c] (fixed summation order)."""
    _on_gpu(x0, grad_base)
    x0 = _prep(x0)
    lows = _same_dtype(x0, [_prep(t) for t in grad_base.unbind(0)])
    return _launch_weight_grad(x0, lows)


@_fake(all_base_b4_12_split_grad_alpha_traceable)
def _(x0: Tensor, grad_base: Tensor) -> Tensor:
    return x0.new_empty((grad_base.shape[0], x0.shape[3], K), dtype=torch.float32)


def _backward_all_base_split(ctx, *grads):
    # local_thc_triton_kernels.py:2655-2663
    if len(grads) == 1 and isinstance(grads[0], (list, tuple)):
        grads = tuple(grads[0])
    x0, alpha_stack = ctx.saved_tensors
    ref = next(g for g in grads if g is not None)
    grad_base = torch.stack([g.contiguous() if g is not None else torch.zeros_like(ref) for g in grads], dim=0)
    need = ctx.needs_input_grad
    grad_x = all_base_b4_12_grad_x_traceable(grad_base, alpha_stack) if need[0] else None
    grad_alpha = all_base_b4_12_split_grad_alpha_traceable(x0, grad_base).to(alpha_stack.dtype) if need[1] else None
    return grad_x, grad_alpha


torch.library.register_autograd(
    all_base_b4_12_split_traceable, _backward_all_base_split, setup_context=_setup_all_base_ctx
)


# ---------------------------------------------------------------------------
# the non-shared lazy schedule (local_thc.py:1491-1512, lthc_v2/model.py:253-268)
# ---------------------------------------------------------------------------
def gamma_matrix(alpha_stack: Tensor, beta_stack: Tensor) -> Tensor:
    """gamma[l, j, c] = sum_k alpha_l[c,k] beta_j[c,k], the same torch expression and dtype as the reference
    (local_thc.py:1496, lthc_v2/model.py:257)."""
    return (alpha_stack[:, None, :, :] * beta_stack[None, :, :, :]).sum(dim=-1)


def triangular_lazy_schedule(x0: Tensor, alpha_stack: Tensor, beta_stack: Tensor, branch) -> Tensor:
    """Run the exact non-shared lazy schedule and return the materialised high-resolution state.

    For l = 0..L-1: z_l = R_l(x0) + sum_{j<l} gamma[l, j] * dz_j, dz_l = branch(l, z_l);
    then x_L = x0 + sum_l P_l(dz_l).  ``alpha_stack`` / ``beta_stack`` are [L, C, 16] in x0's dtype (the
    reference casts them with ``.to(x0.dtype)``); ``branch(l, z)`` returns dz_l of z's shape.  Depth 12
    goes through the reference's 12-pointer active-prefix ops (local_thc.py:1500-1508); other depths up
    to 24 through ``triangular_accumulate_list``.  Every step is differentiable.
    """
    from .ops import final_accumulate_list

    L = alpha_stack.shape[0]
    if beta_stack.shape != alpha_stack.shape:
        raise ValueError(f"alpha_stack {tuple(alpha_stack.shape)} and beta_stack {tuple(beta_stack.shape)} differ")
    bases = all_base_b4_12_split_traceable(x0, alpha_stack.contiguous())
    gamma = gamma_matrix(alpha_stack, beta_stack)
    zero_dz = torch.zeros_like(bases[0]) if L == 12 else None
    dzs: list[Tensor] = []
    for l in range(L):
        z = bases[l]
        if dzs:
            if L == 12:
                dz_args = tuple(dzs[j] if j < l else zero_dz for j in range(12))
                z = triangular_accumulate_b4_12_ptr_active_traceable_ops[l - 1](z, *dz_args, gamma[l].contiguous())
            else:
                z = triangular_accumulate_list(z, list(dzs), gamma[l, :l].contiguous())
        dzs.append(branch(l, z))
    return final_accumulate_list(x0, dzs, list(beta_stack.unbind(0)))


# Reference-style aliases (local_thc.py:30-35 imports these names).
triton_triangular_accumulate_traceable = triangular_accumulate_traceable
triton_triangular_accumulate_b4_12_ptr_traceable = triangular_accumulate_b4_12_ptr_traceable
triton_triangular_active_ops = triangular_accumulate_b4_12_ptr_active_traceable_ops
triton_all_base_b4_12_traceable = all_base_b4_12_traceable
triton_all_base_b4_12_split_traceable = all_base_b4_12_split_traceable
