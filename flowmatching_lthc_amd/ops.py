"""``jit_thc::*`` operators backed by the gfx950 HIP library.

The reference registers its LTHC interface as ``torch.library`` ops in the
``jit_thc`` namespace (flowmatching_lthc/models/local_thc_triton_kernels.py,
via ``triton_op`` + ``register_autograd``).  This module registers the same
names with the same schemas, argument meaning, output dtypes and autograd
formulas, launching hand-written HIP kernels through the C ABI of
``include/lthc.h`` instead of Triton.  The reference's ops are fixed to the
64x64 / 16x16 B/4 geometry; these accept any square grid whose cell side is 4
(so the 128x128 / 32x32 stress shape runs through the same ops).

Every op:
  * runs on CUDA (HIP) tensors only and raises ``ValueError`` for CPU tensors,
    bad shapes, or unsupported dtypes — there is no CPU fallback;
  * allocates its outputs through torch's caching allocator and launches on
    ``torch.cuda.current_stream()`` without host synchronisation, so it can be
    captured in a HIP graph or traced by ``torch.compile`` (``register_fake``);
  * accumulates in fp32 and rounds once to the output dtype.

Naming follows the reference: the legacy "write" op is the algorithmic READ
(high-res -> workspace) and the legacy "read" op is the algorithmic WRITE.
"""

from __future__ import annotations

import functools
import math
import sys
from typing import Callable, Sequence

import torch
from torch import Tensor

from . import _abi

S = 4  # cell side (taps K = 16)
K = S * S


# ---------------------------------------------------------------------------
# torch.compile: every jit_thc op is an opaque Inductor fallback
# ---------------------------------------------------------------------------
_inductor_fallbacks_done = False


def _register_inductor_fallbacks() -> None:
    """Registers every jit_thc op as an Inductor fallback kernel, with the layout constraint its tags give (the
    default: fixed stride order), which is what Inductor does by itself the first time it lowers an op it has no
    lowering for.  Done ahead of time because Inductor's own path formats the op's arguments for a log message
    whatever the log level, and those arguments print their whole producer graph: for the 25-argument
    materialisation, whose dz arguments end chains of twelve blocks of fallback ops, that text grows exponentially
    with the depth and held a compile of the LTHC-B/4 model for many minutes.  Runs once, from the first fake-tensor
    evaluation of a jit_thc op after Inductor's lowering module has been imported (AOTAutograd traces the graph with
    fake tensors after that import and before any lowering); before that, nothing is imported here."""
    global _inductor_fallbacks_done
    if _inductor_fallbacks_done or "torch._inductor.lowering" not in sys.modules:
        return
    _inductor_fallbacks_done = True
    from torch._inductor.lowering import lowerings, make_fallback, tag_to_layout_constraint
    from torch._library.utils import get_layout_constraint_tag

    for name in dir(torch.ops.jit_thc):
        packet = getattr(torch.ops.jit_thc, name)
        if not isinstance(packet, torch._ops.OpOverloadPacket):
            continue
        for overload in packet.overloads():
            op = getattr(packet, overload)
            if op not in lowerings:
                make_fallback(op, layout_constraint=tag_to_layout_constraint(get_layout_constraint_tag(op, with_default=True)))


def _fake(op) -> Callable:
    """Decorator registering `fn` as the fake (meta) implementation of `op` (a custom op, or a "jit_thc::name"
    string for ops defined with torch.library.define), registering the Inductor fallbacks first."""

    def deco(fn: Callable) -> Callable:
        @functools.wraps(fn)
        def fake(*args, **kwargs):
            _register_inductor_fallbacks()
            return fn(*args, **kwargs)

        if isinstance(op, str):
            torch.library.register_fake(op)(fake)
        else:
            op.register_fake(fake)
        return fake

    return deco


# ---------------------------------------------------------------------------
# argument checks
# ---------------------------------------------------------------------------
def _on_gpu(*ts: Tensor) -> None:
    dev = ts[0].device
    if dev.type != "cuda":
        raise ValueError(f"LTHC HIP ops need GPU tensors, got a {dev} tensor (there is no CPU fallback)")
    for t in ts[1:]:
        if t.device != dev:
            raise ValueError(f"all tensors must be on {dev}, got one on {t.device}")


def _prep(t: Tensor) -> Tensor:
    """Contiguous and aligned to 4 elements, as the C ABI requires."""
    t = t.contiguous()
    if t.data_ptr() % (4 * t.element_size()) != 0:
        t = t.clone()
    return t


def _prep_w(w: Tensor, act_dtype: torch.dtype) -> Tensor:
    """Weights in fp32 or the activation dtype (the compiled pairs), contiguous, 16-byte aligned."""
    if w.dtype not in (torch.float32, act_dtype):
        w = w.float()
    w = w.contiguous()
    if w.data_ptr() % 16 != 0:
        w = w.clone()
    return w


def _hi_geom(x: Tensor, name: str = "x") -> tuple[int, int, int]:
    if x.dim() != 4 or x.shape[1] != x.shape[2]:
        raise ValueError(f"{name} must be NHWC [B,H,H,C], got {tuple(x.shape)}")
    b, h, _, c = x.shape
    if h % S != 0:
        raise ValueError(f"{name}: high-res side {h} is not a multiple of the cell side {S}")
    if c % 4 != 0:
        raise ValueError(f"{name}: channels {c} must be a multiple of 4")
    return b, h // S, c


def _lo_geom(z: Tensor, name: str = "z") -> tuple[int, int, int]:
    if z.dim() != 3:
        raise ValueError(f"{name} must be [B,M,C], got {tuple(z.shape)}")
    b, m, c = z.shape
    g = math.isqrt(m)
    if g * g != m:
        raise ValueError(f"{name}: workspace token count {m} is not a square")
    if c % 4 != 0:
        raise ValueError(f"{name}: channels {c} must be a multiple of 4")
    return b, g, c


def _check_weight(w: Tensor, c: int, name: str) -> None:
    if tuple(w.shape) != (c, K):
        raise ValueError(f"{name} must be [{c},{K}], got {tuple(w.shape)}")
    _abi.code(w)


class _NoContext:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NO_CONTEXT = _NoContext()


def _on_device(t: Tensor):
    """Make t's device current for the launch (a no-op context when it already is)."""
    if t.device.index == torch.cuda.current_device():
        return _NO_CONTEXT
    return torch.cuda.device(t.device)


def _same_dtype(ref: Tensor, others: Sequence[Tensor]) -> list[Tensor]:
    return [t if t.dtype == ref.dtype else t.to(ref.dtype) for t in others]


# ---------------------------------------------------------------------------
# launches (inputs already checked and prepared)
# ---------------------------------------------------------------------------
def _launch_read(x: Tensor, w: Tensor, z: Tensor, b: int, g: int, c: int) -> None:
    with _on_device(x):
        rc = _abi.load().lthc_read_fwd(
            x.data_ptr(), _abi.code(x), w.data_ptr(), _abi.code(w), z.data_ptr(), b, g, S, c, _abi.stream_of(x)
        )
    _abi.check(rc, "lthc_read_fwd")


def _launch_materialise(base: Tensor | None, dzs: Sequence[Tensor], betas: Sequence[Tensor], out: Tensor) -> None:
    b, g, c = _lo_geom(dzs[0], "dz")
    wd = _abi.code(betas[0])
    with _on_device(out):
        rc = _abi.load().lthc_materialise_fwd(
            _abi.ptr(base), _abi.ptr_array(dzs), _abi.code(out), _abi.ptr_array(betas), wd, out.data_ptr(),
            b, g, S, c, len(dzs), _abi.stream_of(out),
        )  # fmt: skip
    _abi.check(rc, "lthc_materialise_fwd")


def _launch_read_multi(gr: Tensor, ws: Sequence[Tensor], outs: Sequence[Tensor]) -> None:
    b, g, c = _hi_geom(gr, "grad_out")
    with _on_device(gr):
        rc = _abi.load().lthc_read_multi_fwd(
            gr.data_ptr(), _abi.code(gr), _abi.ptr_array(ws), _abi.code(ws[0]), _abi.ptr_array(outs),
            b, g, S, c, len(ws), _abi.stream_of(gr),
        )  # fmt: skip
    _abi.check(rc, "lthc_read_multi_fwd")


def _launch_weight_grad(high: Tensor, lows: Sequence[Tensor]) -> Tensor:
    b, g, c = _hi_geom(high, "high")
    L = len(lows)
    out = torch.empty((L, c, K), device=high.device, dtype=torch.float32)
    nbytes = _abi.weight_grad_workspace_bytes(b, g, S, c, L)
    ws = torch.empty((max(nbytes, 16),), device=high.device, dtype=torch.uint8)
    with _on_device(high):
        rc = _abi.load().lthc_weight_grad(
            high.data_ptr(), _abi.ptr_array(lows), _abi.code(high), out.data_ptr(), b, g, S, c, L,
            ws.data_ptr(), ws.numel(), _abi.stream_of(high),
        )  # fmt: skip
    _abi.check(rc, "lthc_weight_grad")
    return out


def _launch_materialise_bwd(gr: Tensor, dzs: Sequence[Tensor], betas: Sequence[Tensor], outs: Sequence[Tensor]) -> Tensor:
    """gdZ_l into outs and the fp32 [L,C,16] gbeta from one pass over gr (lthc_materialise_bwd)."""
    b, g, c = _hi_geom(gr, "grad_out")
    L = len(dzs)
    gb = torch.empty((L, c, K), device=gr.device, dtype=torch.float32)
    nbytes = _abi.materialise_bwd_workspace_bytes(b, g, S, c, L)
    ws = torch.empty((max(nbytes, 16),), device=gr.device, dtype=torch.uint8)
    with _on_device(gr):
        rc = _abi.load().lthc_materialise_bwd(
            gr.data_ptr(), _abi.code(gr), _abi.ptr_array(dzs), _abi.ptr_array(betas), _abi.code(betas[0]),
            _abi.ptr_array(outs), gb.data_ptr(), b, g, S, c, L, ws.data_ptr(), ws.numel(), _abi.stream_of(gr),
        )  # fmt: skip
    _abi.check(rc, "lthc_materialise_bwd")
    return gb


@torch.library.custom_op("jit_thc::final_accumulate_backward", mutates_args=())
def final_accumulate_backward(grad_out: Tensor, dzs: list[Tensor], betas: list[Tensor]) -> tuple[Tensor, Tensor]:
    """(gdZ stack [L,B,M,C] in grad_out.dtype, fp32 [L,C,16] gbeta) of X_L = x0 + sum_l P_l(dz_l): the results of
    the two reference backward ops (_grad_dz_ptr, _grad_beta_ptr) from one pass over grad_out."""
    _on_gpu(grad_out, *dzs, *betas)
    b, g, c = _hi_geom(grad_out, "grad_out")
    L = len(dzs)
    if L != len(betas) or not 1 <= L <= _abi.MAX_LAYERS:
        raise ValueError(f"expected 1..{_abi.MAX_LAYERS} dz and as many beta tensors, got {len(dzs)} and {len(betas)}")
    for i, (dz, bt) in enumerate(zip(dzs, betas)):
        if tuple(dz.shape) != (b, g * g, c):
            raise ValueError(f"dz[{i}] must be [{b},{g * g},{c}], got {tuple(dz.shape)}")
        _check_weight(bt, c, f"beta[{i}]")
    grad_out = _prep(grad_out)
    dzs = _same_dtype(grad_out, [_prep(d) for d in dzs])
    betas = [_prep_w(bt, grad_out.dtype) for bt in betas]
    if len({bt.dtype for bt in betas}) != 1:
        betas = [_prep_w(bt.float(), grad_out.dtype) for bt in betas]
    gdz = torch.empty((L, b, g * g, c), device=grad_out.device, dtype=grad_out.dtype)
    gb = _launch_materialise_bwd(grad_out, dzs, betas, list(gdz.unbind(0)))
    return gdz, gb


@_fake(final_accumulate_backward)
def _(grad_out: Tensor, dzs: list[Tensor], betas: list[Tensor]):
    b, g, c = _hi_geom(grad_out, "grad_out")
    return grad_out.new_empty((len(dzs), b, g * g, c)), grad_out.new_empty((len(dzs), c, K), dtype=torch.float32)


# ---------------------------------------------------------------------------
# READ  (jit_thc::local_write_traceable, local_thc_triton_kernels.py:2673-2683)
# ---------------------------------------------------------------------------
@torch.library.custom_op("jit_thc::local_write_traceable", mutates_args=())
def local_write_traceable(x: Tensor, weight: Tensor) -> Tensor:
    """Z[b,m,c] = sum_k weight[c,k] X[b,m,k,c]: x [B,H,H,C] -> z [B,(H/4)^2,C] in x.dtype."""
    _on_gpu(x, weight)
    b, g, c = _hi_geom(x)
    _check_weight(weight, c, "weight")
    x = _prep(x)
    w = _prep_w(weight, x.dtype)
    z = torch.empty((b, g * g, c), device=x.device, dtype=x.dtype)
    _launch_read(x, w, z, b, g, c)
    return z


@_fake(local_write_traceable)
def _(x: Tensor, weight: Tensor) -> Tensor:
    b, g, c = _hi_geom(x)
    return x.new_empty((b, g * g, c))


# ---------------------------------------------------------------------------
# WRITE  (jit_thc::local_read_traceable, local_thc_triton_kernels.py:2686-2696)
# ---------------------------------------------------------------------------
@torch.library.custom_op("jit_thc::local_read_traceable", mutates_args=())
def local_read_traceable(z: Tensor, weight: Tensor) -> Tensor:
    """X[b,m,k,c] = weight[c,k] Z[b,m,c]: z [B,M,C] -> x [B,4*sqrt(M),4*sqrt(M),C] in z.dtype."""
    _on_gpu(z, weight)
    b, g, c = _lo_geom(z)
    _check_weight(weight, c, "weight")
    z = _prep(z)
    w = _prep_w(weight, z.dtype)
    out = torch.empty((b, g * S, g * S, c), device=z.device, dtype=z.dtype)
    _launch_materialise(None, [z], [w], out)
    return out


@_fake(local_read_traceable)
def _(z: Tensor, weight: Tensor) -> Tensor:
    b, g, c = _lo_geom(z)
    return z.new_empty((b, g * S, g * S, c))


# ---------------------------------------------------------------------------
# CELL WEIGHT GRADIENT  (jit_thc::local_weight_grad_traceable, :2699-2710)
# ---------------------------------------------------------------------------
@torch.library.custom_op("jit_thc::local_weight_grad_traceable", mutates_args=())
def local_weight_grad_traceable(high: Tensor, low: Tensor) -> Tensor:
    """gW[c,k] = sum_{b,m} high[b,m,k,c] low[b,m,c] in fp32 [C,16] (deterministic order)."""
    _on_gpu(high, low)
    b, g, c = _hi_geom(high, "high")
    bl, gl, cl = _lo_geom(low, "low")
    if (bl, gl, cl) != (b, g, c):
        raise ValueError(f"high {tuple(high.shape)} and low {tuple(low.shape)} do not match")
    high = _prep(high)
    (low,) = _same_dtype(high, [_prep(low)])
    return _launch_weight_grad(high, [low])[0]


@_fake(local_weight_grad_traceable)
def _(high: Tensor, low: Tensor) -> Tensor:
    c = high.shape[3]
    return high.new_empty((c, K), dtype=torch.float32)


def _setup_write_ctx(ctx, inputs, output):
    x, weight = inputs
    ctx.save_for_backward(x, weight)


def _backward_write(ctx, grad_z):
    # local_thc_triton_kernels.py:2726-2729
    x, weight = ctx.saved_tensors
    grad_x = local_read_traceable(grad_z, weight) if ctx.needs_input_grad[0] else None
    grad_w = local_weight_grad_traceable(x, grad_z).to(dtype=weight.dtype) if ctx.needs_input_grad[1] else None
    return grad_x, grad_w


def _setup_read_ctx(ctx, inputs, output):
    z, weight = inputs
    ctx.save_for_backward(z, weight)


def _backward_read(ctx, grad_x):
    # local_thc_triton_kernels.py:2737-2741
    z, weight = ctx.saved_tensors
    grad_z = local_write_traceable(grad_x, weight) if ctx.needs_input_grad[0] else None
    grad_w = local_weight_grad_traceable(grad_x, z).to(dtype=weight.dtype) if ctx.needs_input_grad[1] else None
    return grad_z, grad_w


torch.library.register_autograd(local_write_traceable, _backward_write, setup_context=_setup_write_ctx)
torch.library.register_autograd(local_read_traceable, _backward_read, setup_context=_setup_read_ctx)


# ---------------------------------------------------------------------------
# WRITE-ADD  (jit_thc::local_read_add_traceable, local_thc_triton_kernels.py:2713-2723)
# ---------------------------------------------------------------------------
@torch.library.custom_op("jit_thc::local_read_add_traceable", mutates_args=())
def local_read_add_traceable(z: Tensor, weight: Tensor, x: Tensor) -> Tensor:
    """x[b,m,k,c] + weight[c,k] z[b,m,c] in x.dtype, one pass over x (the materialisation with L = 1)."""
    _on_gpu(z, weight, x)
    b, g, c = _lo_geom(z)
    bx, gx, cx = _hi_geom(x)
    if (bx, gx, cx) != (b, g, c):
        raise ValueError(f"z {tuple(z.shape)} and x {tuple(x.shape)} do not describe the same cells")
    _check_weight(weight, c, "weight")
    x = _prep(x)
    (z,) = _same_dtype(x, [_prep(z)])
    w = _prep_w(weight, x.dtype)
    out = torch.empty_like(x)
    _launch_materialise(x, [z], [w], out)
    return out


@_fake(local_read_add_traceable)
def _(z: Tensor, weight: Tensor, x: Tensor) -> Tensor:
    return torch.empty_like(x)


def _setup_read_add_ctx(ctx, inputs, output):
    z, weight, _ = inputs
    ctx.save_for_backward(z, weight)


def _backward_read_add(ctx, grad_out):
    # local_thc_triton_kernels.py:2749-2754
    z, weight = ctx.saved_tensors
    grad_z = local_write_traceable(grad_out, weight) if ctx.needs_input_grad[0] else None
    grad_w = local_weight_grad_traceable(grad_out, z).to(dtype=weight.dtype) if ctx.needs_input_grad[1] else None
    return grad_z, grad_w, grad_out


torch.library.register_autograd(local_read_add_traceable, _backward_read_add, setup_context=_setup_read_add_ctx)


# ---------------------------------------------------------------------------
# Legacy per-block functions (local_thc_triton_kernels.py:1379-1575): the same
# maps as the ops above, plus "frozen" forms whose weights get no gradient
# ---------------------------------------------------------------------------
class _ReadNoWeightGrad(torch.autograd.Function):
    """z = R_weight(x); backward dX = R^T(gz) only (_LocalWriteNoWeightGradFunction, :1417-1447)."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor) -> Tensor:
        ctx.save_for_backward(weight)
        return local_write_traceable(x, weight)

    @staticmethod
    def backward(ctx, grad_z: Tensor):
        (weight,) = ctx.saved_tensors
        return local_read_traceable(grad_z.contiguous(), weight), None


class _WriteAddNoWeightGrad(torch.autograd.Function):
    """x + P_weight(z); backward (R(g), None, g) (_LocalReadAddNoWeightGradFunction, :1525-1555)."""

    @staticmethod
    def forward(ctx, z: Tensor, weight: Tensor, x: Tensor) -> Tensor:
        ctx.save_for_backward(weight)
        return local_read_add_traceable(z, weight, x)

    @staticmethod
    def backward(ctx, grad_out: Tensor):
        (weight,) = ctx.saved_tensors
        grad_out = grad_out.contiguous()
        return local_write_traceable(grad_out, weight), None, grad_out


def local_write(x: Tensor, weight: Tensor) -> Tensor:
    """The read R_weight(x) with gradients for x and weight (local_thc_triton_kernels.py:1558-1559)."""
    return local_write_traceable(x, weight)


def local_read(z: Tensor, weight: Tensor) -> Tensor:
    """The write P_weight(z) with gradients for z and weight (:1562-1563)."""
    return local_read_traceable(z, weight)


def local_write_no_weight_grad(x: Tensor, weight: Tensor) -> Tensor:
    """The read with a frozen weight: no weight gradient (:1566-1567)."""
    return _ReadNoWeightGrad.apply(x, weight)


def local_read_add(z: Tensor, weight: Tensor, x: Tensor) -> Tensor:
    """x + P_weight(z) in one pass, gradients for all three (:1570-1571)."""
    return local_read_add_traceable(z, weight, x)


def local_read_add_no_weight_grad(z: Tensor, weight: Tensor, x: Tensor) -> Tensor:
    """x + P_weight(z) with a frozen weight (:1574-1575)."""
    return _WriteAddNoWeightGrad.apply(z, weight, x)


class _OpenInterface(torch.autograd.Function):
    """(x, Z0 = R(x)) as one autograd node.

    In the lazy forward x feeds both the read and the final materialisation,
    so autograd would write R^T(gZ0) as a full high-res tensor and then add
    the materialisation's gradient to it (two more passes over x's size).
    Here the node receives both gradients together and returns
    dX = g_x + R^T(gZ0) from one local_read_add pass; dW = sum x * gZ0.
    """

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor):
        z = local_write_traceable(x, weight)
        ctx.save_for_backward(x, weight)
        ctx.set_materialize_grads(False)  # an unused output's gradient arrives as None, not zeros
        return x.view_as(x), z

    @staticmethod
    def backward(ctx, grad_x: Tensor | None, grad_z: Tensor | None):
        x, weight = ctx.saved_tensors
        gx = gw = None
        if grad_z is None:
            gx = grad_x
        else:
            if ctx.needs_input_grad[0]:
                if grad_x is None:
                    gx = local_read_traceable(grad_z, weight)
                else:
                    gx = local_read_add_traceable(grad_z, weight, grad_x.to(x.dtype))
            if ctx.needs_input_grad[1]:
                gw = local_weight_grad_traceable(x, grad_z).to(dtype=weight.dtype)
        return gx, gw


def read_with_residual(x: Tensor, weight: Tensor) -> tuple[Tensor, Tensor]:
    """(x, local_write_traceable(x, weight)) with a fused backward for a later consumer of x.

    Values are those of the two separate uses; the backward of x is
    g_x + R^T(gZ) in one pass instead of autograd's separate write and add.
    """
    return _OpenInterface.apply(x, weight)


# ---------------------------------------------------------------------------
# MATERIALISE, stacked form (jit_thc::final_accumulate_b4_traceable, :1578-1666)
# ---------------------------------------------------------------------------
def _check_stack(x0: Tensor, dz_stack: Tensor, beta_stack: Tensor) -> tuple[int, int, int, int]:
    b, g, c = _hi_geom(x0, "x0")
    if dz_stack.dim() != 4 or tuple(dz_stack.shape[1:]) != (b, g * g, c):
        raise ValueError(f"dz_stack must be [L,{b},{g * g},{c}], got {tuple(dz_stack.shape)}")
    L = dz_stack.shape[0]
    if tuple(beta_stack.shape) != (L, c, K):
        raise ValueError(f"beta_stack must be [{L},{c},{K}], got {tuple(beta_stack.shape)}")
    if not 1 <= L <= _abi.MAX_LAYERS:
        raise ValueError(f"depth {L} outside 1..{_abi.MAX_LAYERS}")
    return b, g, c, L


@torch.library.custom_op("jit_thc::final_accumulate_b4_traceable", mutates_args=())
def final_accumulate_b4_traceable(x0: Tensor, dz_stack: Tensor, beta_stack: Tensor) -> Tensor:
    """X_L = x0 + sum_l beta_stack[l][c,k] dz_stack[l][b,m,c] in x0.dtype."""
    _on_gpu(x0, dz_stack, beta_stack)
    _check_stack(x0, dz_stack, beta_stack)
    x0 = _prep(x0)
    (dz_stack,) = _same_dtype(x0, [_prep(dz_stack)])
    beta_stack = _prep_w(beta_stack, x0.dtype)
    out = torch.empty_like(x0)
    _launch_materialise(x0, list(dz_stack.unbind(0)), list(beta_stack.unbind(0)), out)
    return out


@_fake(final_accumulate_b4_traceable)
def _(x0: Tensor, dz_stack: Tensor, beta_stack: Tensor) -> Tensor:
    return torch.empty_like(x0)


@torch.library.custom_op("jit_thc::final_accumulate_b4_grad_dz", mutates_args=())
def final_accumulate_b4_grad_dz_traceable(grad_out: Tensor, beta_stack: Tensor) -> Tensor:
    """gdZ[l,b,m,c] = sum_k beta_stack[l][c,k] grad_out[b,m,k,c] in grad_out.dtype ([L,B,M,C])."""
    _on_gpu(grad_out, beta_stack)
    b, g, c = _hi_geom(grad_out, "grad_out")
    L = beta_stack.shape[0]
    if beta_stack.dim() != 3 or tuple(beta_stack.shape[1:]) != (c, K) or not 1 <= L <= _abi.MAX_LAYERS:
        raise ValueError(f"beta_stack must be [L,{c},{K}] with 1 <= L <= {_abi.MAX_LAYERS}, got {tuple(beta_stack.shape)}")
    grad_out = _prep(grad_out)
    beta_stack = _prep_w(beta_stack, grad_out.dtype)
    gdz = torch.empty((L, b, g * g, c), device=grad_out.device, dtype=grad_out.dtype)
    _launch_read_multi(grad_out, list(beta_stack.unbind(0)), list(gdz.unbind(0)))
    return gdz


@_fake(final_accumulate_b4_grad_dz_traceable)
def _(grad_out: Tensor, beta_stack: Tensor) -> Tensor:
    b, g, c = _hi_geom(grad_out, "grad_out")
    return grad_out.new_empty((beta_stack.shape[0], b, g * g, c))


@torch.library.custom_op("jit_thc::final_accumulate_b4_grad_beta", mutates_args=())
def final_accumulate_b4_grad_beta_traceable(grad_out: Tensor, dz_stack: Tensor, beta_stack: Tensor) -> Tensor:
    """gbeta[l,c,k] = sum_{b,m} grad_out[b,m,k,c] dz_stack[l][b,m,c] in fp32 [L,C,16]."""
    _on_gpu(grad_out, dz_stack, beta_stack)
    _check_stack(grad_out, dz_stack, beta_stack)
    grad_out = _prep(grad_out)
    (dz_stack,) = _same_dtype(grad_out, [_prep(dz_stack)])
    return _launch_weight_grad(grad_out, list(dz_stack.unbind(0)))


@_fake(final_accumulate_b4_grad_beta_traceable)
def _(grad_out: Tensor, dz_stack: Tensor, beta_stack: Tensor) -> Tensor:
    return grad_out.new_empty((dz_stack.shape[0], grad_out.shape[3], K), dtype=torch.float32)


def _setup_final_accumulate_ctx(ctx, inputs, output):
    _, dz_stack, beta_stack = inputs
    ctx.save_for_backward(dz_stack, beta_stack)


def _backward_final_accumulate(ctx, grad_out):
    # local_thc_triton_kernels.py:1652-1660: grad_x0 is grad_out itself.
    dz_stack, beta_stack = ctx.saved_tensors
    grad_out = grad_out.contiguous()
    if ctx.needs_input_grad[1] and ctx.needs_input_grad[2]:  # both from one pass over grad_out
        grad_dz, gb = final_accumulate_backward(grad_out, list(dz_stack.unbind(0)), list(beta_stack.unbind(0)))
        return grad_out, grad_dz, gb.to(dtype=beta_stack.dtype)
    grad_dz = final_accumulate_b4_grad_dz_traceable(grad_out, beta_stack) if ctx.needs_input_grad[1] else None
    grad_beta = None
    if ctx.needs_input_grad[2]:
        grad_beta = final_accumulate_b4_grad_beta_traceable(grad_out, dz_stack, beta_stack).to(dtype=beta_stack.dtype)
    return grad_out, grad_dz, grad_beta


torch.library.register_autograd(
    final_accumulate_b4_traceable, _backward_final_accumulate, setup_context=_setup_final_accumulate_ctx
)


# ---------------------------------------------------------------------------
# MATERIALISE, any depth as a list of layers (no reference op: the reference's
# generic path is the Python write_add loop of local_thc.py:1368-1372, and its
# stacked op is fixed to the 64x64 / 16x16 geometry)
# ---------------------------------------------------------------------------
def _check_list(x0: Tensor, dzs: Sequence[Tensor], betas: Sequence[Tensor]) -> int:
    b, g, c = _hi_geom(x0, "x0")
    L = len(dzs)
    if L != len(betas) or not 1 <= L <= _abi.MAX_LAYERS:
        raise ValueError(f"expected 1..{_abi.MAX_LAYERS} dz and as many beta tensors, got {len(dzs)} and {len(betas)}")
    for i, (dz, bt) in enumerate(zip(dzs, betas)):
        if tuple(dz.shape) != (b, g * g, c):
            raise ValueError(f"dz[{i}] must be [{b},{g * g},{c}], got {tuple(dz.shape)}")
        _check_weight(bt, c, f"beta[{i}]")
    return L


@torch.library.custom_op("jit_thc::final_accumulate_list", mutates_args=())
def final_accumulate_list(x0: Tensor, dzs: list[Tensor], betas: list[Tensor]) -> Tensor:
    """X_L = x0 + sum_l betas[l][c,k] dzs[l][b,m,c] in x0.dtype, one pass, the L layers passed as lists."""
    _on_gpu(x0, *dzs, *betas)
    _check_list(x0, dzs, betas)
    x0 = _prep(x0)
    dzs = _same_dtype(x0, [_prep(d) for d in dzs])
    betas = [_prep_w(bt, x0.dtype) for bt in betas]
    if len({bt.dtype for bt in betas}) != 1:
        betas = [bt.float() for bt in betas]
    out = torch.empty_like(x0)
    _launch_materialise(x0, dzs, betas, out)
    return out


@_fake(final_accumulate_list)
def _(x0: Tensor, dzs: list[Tensor], betas: list[Tensor]) -> Tensor:
    return torch.empty_like(x0)


@torch.library.custom_op("jit_thc::final_accumulate_list_grad_dz", mutates_args=())
def final_accumulate_list_grad_dz(grad_out: Tensor, betas: list[Tensor]) -> list[Tensor]:
    """gdZ_l[b,m,c] = sum_k betas[l][c,k] grad_out[b,m,k,c], one tensor per layer, in grad_out.dtype."""
    _on_gpu(grad_out, *betas)
    b, g, c = _hi_geom(grad_out, "grad_out")
    for i, bt in enumerate(betas):
        _check_weight(bt, c, f"beta[{i}]")
    grad_out = _prep(grad_out)
    betas = [_prep_w(bt, grad_out.dtype) for bt in betas]
    if len({bt.dtype for bt in betas}) != 1:
        betas = [bt.float() for bt in betas]
    outs = [torch.empty((b, g * g, c), device=grad_out.device, dtype=grad_out.dtype) for _ in betas]
    _launch_read_multi(grad_out, betas, outs)
    return outs


@_fake(final_accumulate_list_grad_dz)
def _(grad_out: Tensor, betas: list[Tensor]) -> list[Tensor]:
    b, g, c = _hi_geom(grad_out, "grad_out")
    return [grad_out.new_empty((b, g * g, c)) for _ in betas]


@torch.library.custom_op("jit_thc::final_accumulate_list_grad_beta", mutates_args=())
def final_accumulate_list_grad_beta(grad_out: Tensor, dzs: list[Tensor]) -> Tensor:
    """gbeta[l,c,k] = sum_{b,m} grad_out[b,m,k,c] dzs[l][b,m,c] in fp32 [L,C,16] (deterministic order)."""
    _on_gpu(grad_out, *dzs)
    b, g, c = _hi_geom(grad_out, "grad_out")
    for i, dz in enumerate(dzs):
        if tuple(dz.shape) != (b, g * g, c):
            raise ValueError(f"dz[{i}] must be [{b},{g * g},{c}], got {tuple(dz.shape)}")
    grad_out = _prep(grad_out)
    dzs = _same_dtype(grad_out, [_prep(d) for d in dzs])
    return _launch_weight_grad(grad_out, dzs)


@_fake(final_accumulate_list_grad_beta)
def _(grad_out: Tensor, dzs: list[Tensor]) -> Tensor:
    return grad_out.new_empty((len(dzs), grad_out.shape[3], K), dtype=torch.float32)


def _setup_final_accumulate_list_ctx(ctx, inputs, output):
    _, dzs, betas = inputs
    ctx.save_for_backward(*dzs, *betas)
    ctx.L = len(dzs)


def _backward_final_accumulate_list(ctx, grad_out):
    saved = ctx.saved_tensors
    dzs, betas = saved[: ctx.L], saved[ctx.L :]
    grad_out = grad_out.contiguous()
    if ctx.needs_input_grad[1] and ctx.needs_input_grad[2]:  # both from one pass over grad_out
        gdz, gb = final_accumulate_backward(grad_out, list(dzs), list(betas))
        return grad_out, list(gdz.unbind(0)), [g.to(dtype=bt.dtype) for g, bt in zip(gb.unbind(0), betas, strict=True)]
    grad_dzs = final_accumulate_list_grad_dz(grad_out, list(betas)) if ctx.needs_input_grad[1] else None
    grad_betas = None
    if ctx.needs_input_grad[2]:
        gb = final_accumulate_list_grad_beta(grad_out, list(dzs))
        grad_betas = [g.to(dtype=bt.dtype) for g, bt in zip(gb.unbind(0), betas, strict=True)]
    return grad_out, grad_dzs, grad_betas


torch.library.register_autograd(
    final_accumulate_list, _backward_final_accumulate_list, setup_context=_setup_final_accumulate_list_ctx
)


# ---------------------------------------------------------------------------
# MATERIALISE, 12 separate layers (jit_thc::final_accumulate_b4_12_traceable,
# local_thc_triton_kernels.py:1669-1736) and its backward ops (:1800-1919)
# ---------------------------------------------------------------------------
def _check_12(x0: Tensor, dzs: Sequence[Tensor], betas: Sequence[Tensor]) -> None:
    b, g, c = _hi_geom(x0, "x0")
    for i, dz in enumerate(dzs):
        if tuple(dz.shape) != (b, g * g, c):
            raise ValueError(f"dz{i} must be [{b},{g * g},{c}], got {tuple(dz.shape)}")
    for i, bt in enumerate(betas):
        _check_weight(bt, c, f"beta{i}")


@torch.library.custom_op("jit_thc::final_accumulate_b4_12_traceable", mutates_args=())
def final_accumulate_b4_12_traceable(
    x0: Tensor,
    dz0: Tensor, dz1: Tensor, dz2: Tensor, dz3: Tensor, dz4: Tensor, dz5: Tensor,
    dz6: Tensor, dz7: Tensor, dz8: Tensor, dz9: Tensor, dz10: Tensor, dz11: Tensor,
    beta0: Tensor, beta1: Tensor, beta2: Tensor, beta3: Tensor, beta4: Tensor, beta5: Tensor,
    beta6: Tensor, beta7: Tensor, beta8: Tensor, beta9: Tensor, beta10: Tensor, beta11: Tensor,
) -> Tensor:  # fmt: skip
    """X_L = x0 + sum_{l<12} beta_l[c,k] dz_l[b,m,c]; one pass over X0, stored once in x0.dtype."""
    dzs = [dz0, dz1, dz2, dz3, dz4, dz5, dz6, dz7, dz8, dz9, dz10, dz11]
    betas = [beta0, beta1, beta2, beta3, beta4, beta5, beta6, beta7, beta8, beta9, beta10, beta11]
    _on_gpu(x0, *dzs, *betas)
    _check_12(x0, dzs, betas)
    x0 = _prep(x0)
    dzs = _same_dtype(x0, [_prep(d) for d in dzs])
    betas = [_prep_w(bt, x0.dtype) for bt in betas]
    if len({bt.dtype for bt in betas}) != 1:
        betas = [_prep_w(bt.float(), x0.dtype) for bt in betas]
    out = torch.empty_like(x0)
    _launch_materialise(x0, dzs, betas, out)
    return out


@_fake(final_accumulate_b4_12_traceable)
def _(x0, *rest):
    return torch.empty_like(x0)


@torch.library.custom_op("jit_thc::final_accumulate_b4_12_grad_dz_ptr", mutates_args=())
def final_accumulate_b4_12_grad_dz_ptr_traceable(
    grad_out: Tensor,
    beta0: Tensor, beta1: Tensor, beta2: Tensor, beta3: Tensor, beta4: Tensor, beta5: Tensor,
    beta6: Tensor, beta7: Tensor, beta8: Tensor, beta9: Tensor, beta10: Tensor, beta11: Tensor,
) -> Tensor:  # fmt: skip
    """[12,B,M,C] stack of gdZ_l = sum_k beta_l[c,k] grad_out[b,m,k,c] in grad_out.dtype."""
    betas = [beta0, beta1, beta2, beta3, beta4, beta5, beta6, beta7, beta8, beta9, beta10, beta11]
    _on_gpu(grad_out, *betas)
    b, g, c = _hi_geom(grad_out, "grad_out")
    for i, bt in enumerate(betas):
        _check_weight(bt, c, f"beta{i}")
    grad_out = _prep(grad_out)
    betas = [_prep_w(bt, grad_out.dtype) for bt in betas]
    if len({bt.dtype for bt in betas}) != 1:
        betas = [_prep_w(bt.float(), grad_out.dtype) for bt in betas]
    gdz = torch.empty((12, b, g * g, c), device=grad_out.device, dtype=grad_out.dtype)
    _launch_read_multi(grad_out, betas, list(gdz.unbind(0)))
    return gdz


@_fake(final_accumulate_b4_12_grad_dz_ptr_traceable)
def _(grad_out, *betas):
    b, g, c = _hi_geom(grad_out, "grad_out")
    return grad_out.new_empty((12, b, g * g, c))


@torch.library.custom_op("jit_thc::final_accumulate_b4_12_grad_beta_ptr", mutates_args=())
def final_accumulate_b4_12_grad_beta_ptr_traceable(
    grad_out: Tensor,
    dz0: Tensor, dz1: Tensor, dz2: Tensor, dz3: Tensor, dz4: Tensor, dz5: Tensor,
    dz6: Tensor, dz7: Tensor, dz8: Tensor, dz9: Tensor, dz10: Tensor, dz11: Tensor,
) -> Tensor:  # fmt: skip
    """fp32 [12,C,16] stack of gbeta_l = sum_{b,m} grad_out[b,m,k,c] dz_l[b,m,c] (deterministic)."""
    dzs = [dz0, dz1, dz2, dz3, dz4, dz5, dz6, dz7, dz8, dz9, dz10, dz11]
    _on_gpu(grad_out, *dzs)
    b, g, c = _hi_geom(grad_out, "grad_out")
    for i, dz in enumerate(dzs):
        if tuple(dz.shape) != (b, g * g, c):
            raise ValueError(f"dz{i} must be [{b},{g * g},{c}], got {tuple(dz.shape)}")
    grad_out = _prep(grad_out)
    dzs = _same_dtype(grad_out, [_prep(d) for d in dzs])
    return _launch_weight_grad(grad_out, dzs)


@_fake(final_accumulate_b4_12_grad_beta_ptr_traceable)
def _(grad_out, *dzs):
    return grad_out.new_empty((12, grad_out.shape[3], K), dtype=torch.float32)


def _setup_final_accumulate_12_ctx(ctx, inputs, output):
    ctx.save_for_backward(*inputs[1:])


def _backward_final_accumulate_12(ctx, grad_out):
    # local_thc_triton_kernels.py:1901-1912: grad_x0 is grad_out itself.
    saved = ctx.saved_tensors
    dzs, betas = saved[:12], saved[12:]
    grad_out = grad_out.contiguous()
    need = ctx.needs_input_grad
    grad_dzs = (None,) * 12
    grad_betas = (None,) * 12
    if any(need[1:13]) and any(need[13:25]):  # both from one pass over grad_out
        gdz, gb = final_accumulate_backward(grad_out, list(dzs), list(betas))
        grad_betas = tuple(g.to(dtype=bt.dtype) for g, bt in zip(gb.unbind(0), betas, strict=True))
        return (grad_out, *gdz.unbind(0), *grad_betas)
    if any(need[1:13]):
        grad_dzs = tuple(final_accumulate_b4_12_grad_dz_ptr_traceable(grad_out, *betas).unbind(0))
    if any(need[13:25]):
        gb = final_accumulate_b4_12_grad_beta_ptr_traceable(grad_out, *dzs)
        grad_betas = tuple(g.to(dtype=bt.dtype) for g, bt in zip(gb.unbind(0), betas, strict=True))
    return (grad_out, *grad_dzs, *grad_betas)


torch.library.register_autograd(
    final_accumulate_b4_12_traceable, _backward_final_accumulate_12, setup_context=_setup_final_accumulate_12_ctx
)


# ---------------------------------------------------------------------------
# LAZY WORKSPACE RECURRENCE  (no reference op: local_thc.py:1325-1328 is eager torch)
# ---------------------------------------------------------------------------
def _check_recur(z: Tensor, dz: Tensor, gamma: Tensor) -> int:
    if z.shape != dz.shape or z.dim() < 1:
        raise ValueError(f"z {tuple(z.shape)} and dz {tuple(dz.shape)} must have the same shape")
    c = z.shape[-1]
    if tuple(gamma.shape) != (c,):
        raise ValueError(f"gamma must be [{c}], got {tuple(gamma.shape)}")
    if c % 4 != 0:
        raise ValueError(f"channels {c} must be a multiple of 4")
    _abi.code(gamma)
    return c


@torch.library.custom_op("jit_thc::lazy_workspace_update", mutates_args=())
def lazy_workspace_update(z: Tensor, dz: Tensor, gamma: Tensor) -> Tensor:
    """Z_{l+1} = Z_l + gamma[c] * dZ_l computed as fma(gamma, dz, z), in the promoted dtype of z and dz."""
    _on_gpu(z, dz, gamma)
    c = _check_recur(z, dz, gamma)
    dt = torch.promote_types(z.dtype, dz.dtype)
    z, dz, gamma = _prep(z.to(dt)), _prep(dz.to(dt)), _prep(gamma)
    out = torch.empty_like(z)
    with _on_device(z):
        rc = _abi.load().lthc_recur_fwd(
            z.data_ptr(), dz.data_ptr(), _abi.code(z), gamma.data_ptr(), _abi.code(gamma), out.data_ptr(),
            z.numel() // c, c, _abi.stream_of(z),
        )  # fmt: skip
    _abi.check(rc, "lthc_recur_fwd")
    return out


@_fake(lazy_workspace_update)
def _(z: Tensor, dz: Tensor, gamma: Tensor) -> Tensor:
    return z.new_empty(z.shape, dtype=torch.promote_types(z.dtype, dz.dtype))


@torch.library.custom_op("jit_thc::lazy_workspace_update_backward", mutates_args=())
def lazy_workspace_update_backward(
    grad: Tensor, dz: Tensor, gamma: Tensor, gdz_add: Tensor | None = None
) -> tuple[Tensor, Tensor]:
    """(gamma * grad [+ gdz_add] in grad.dtype, fp32 [C] sum over rows of grad * dz)."""
    _on_gpu(grad, dz, gamma)
    c = _check_recur(grad, dz, gamma)
    grad = _prep(grad)
    (dz,) = _same_dtype(grad, [_prep(dz)])
    if gdz_add is not None:
        if gdz_add.shape != grad.shape:
            raise ValueError(f"gdz_add {tuple(gdz_add.shape)} must match grad {tuple(grad.shape)}")
        (gdz_add,) = _same_dtype(grad, [_prep(gdz_add)])
    gamma = _prep(gamma)
    rows = grad.numel() // c
    gdz = torch.empty_like(grad)
    ggamma = torch.empty((c,), device=grad.device, dtype=torch.float32)
    ws = torch.empty((max(_abi.recur_bwd_workspace_bytes(rows, c), 16),), device=grad.device, dtype=torch.uint8)
    with _on_device(grad):
        rc = _abi.load().lthc_recur_bwd(
            grad.data_ptr(), dz.data_ptr(), _abi.ptr(gdz_add), _abi.code(grad), gamma.data_ptr(), _abi.code(gamma),
            gdz.data_ptr(), ggamma.data_ptr(), rows, c, ws.data_ptr(), ws.numel(), _abi.stream_of(grad),
        )  # fmt: skip
    _abi.check(rc, "lthc_recur_bwd")
    return gdz, ggamma


@_fake(lazy_workspace_update_backward)
def _(grad: Tensor, dz: Tensor, gamma: Tensor, gdz_add: Tensor | None = None):
    return torch.empty_like(grad), grad.new_empty((grad.shape[-1],), dtype=torch.float32)


@torch.library.custom_op("jit_thc::lazy_workspace_update_backward_sum", mutates_args=())
def lazy_workspace_update_backward_sum(
    grad: Tensor, grad_branch: Tensor, dz: Tensor, gamma: Tensor, gdz_add: Tensor | None = None
) -> tuple[Tensor, Tensor, Tensor]:
    """(g = grad + grad_branch rounded to grad.dtype, gamma * g [+ gdz_add], [C] sum over rows of g * dz in fp32,
    rounded once to gamma's dtype): lazy_workspace_update_backward of the two gradients of z_next, summed in the
    same pass."""
    _on_gpu(grad, grad_branch, dz, gamma)
    c = _check_recur(grad, dz, gamma)
    if grad_branch.shape != grad.shape:
        raise ValueError(f"grad_branch {tuple(grad_branch.shape)} must match grad {tuple(grad.shape)}")
    grad = _prep(grad)
    dz, grad_branch = _same_dtype(grad, [_prep(dz), _prep(grad_branch)])
    if gdz_add is not None:
        if gdz_add.shape != grad.shape:
            raise ValueError(f"gdz_add {tuple(gdz_add.shape)} must match grad {tuple(grad.shape)}")
        (gdz_add,) = _same_dtype(grad, [_prep(gdz_add)])
    gamma = _prep(gamma)
    rows = grad.numel() // c
    gsum = torch.empty_like(grad)
    gdz = torch.empty_like(grad)
    ggamma = torch.empty((c,), device=grad.device, dtype=gamma.dtype)
    ws = torch.empty((max(_abi.recur_bwd_workspace_bytes(rows, c), 16),), device=grad.device, dtype=torch.uint8)
    with _on_device(grad):
        rc = _abi.load().lthc_recur_bwd_sum(
            grad.data_ptr(), grad_branch.data_ptr(), dz.data_ptr(), _abi.ptr(gdz_add), _abi.code(grad),
            gamma.data_ptr(), _abi.code(gamma), gsum.data_ptr(), gdz.data_ptr(), ggamma.data_ptr(), _abi.code(ggamma),
            rows, c, ws.data_ptr(), ws.numel(), _abi.stream_of(grad),
        )  # fmt: skip
    _abi.check(rc, "lthc_recur_bwd_sum")
    return gsum, gdz, ggamma


@_fake(lazy_workspace_update_backward_sum)
def _(grad: Tensor, grad_branch: Tensor, dz: Tensor, gamma: Tensor, gdz_add: Tensor | None = None):
    return torch.empty_like(grad), torch.empty_like(grad), grad.new_empty((grad.shape[-1],), dtype=gamma.dtype)


def _setup_recur_ctx(ctx, inputs, output):
    _, dz, gamma = inputs
    ctx.save_for_backward(dz, gamma)
    ctx.z_dtype = inputs[0].dtype


def _backward_recur(ctx, grad):
    dz, gamma = ctx.saved_tensors
    need = ctx.needs_input_grad
    grad_z = grad.to(ctx.z_dtype) if need[0] else None
    grad_dz = grad_gamma = None
    if need[1] or need[2]:
        gdz, gg = lazy_workspace_update_backward(grad, dz, gamma)
        grad_dz = gdz.to(dz.dtype) if need[1] else None
        grad_gamma = gg.to(gamma.dtype) if need[2] else None
    return grad_z, grad_dz, grad_gamma


torch.library.register_autograd(lazy_workspace_update, _backward_recur, setup_context=_setup_recur_ctx)


class _RecurStep(torch.autograd.Function):
    """(Z_{l+1} = Z_l + gamma * dZ_l, dZ_l) as one autograd node, or (Z_{l+1}, Z_{l+1}', dZ_l) with `split`.

    In the lazy forward dZ_l feeds both the recurrence and the final
    materialisation, so autograd would add the two gradients of dZ_l in a
    separate pass; here the node receives both and one recurrence-backward
    launch writes gamma * g + (materialisation's gradient).  With `split`,
    Z_{l+1} is returned twice, one for the next recurrence step and one for
    the next block's branch: the node then also receives Z_{l+1}'s two
    gradients apart and sums them in the same launch, where autograd would
    add them in a pass of its own.
    """

    @staticmethod
    def forward(ctx, z: Tensor, dz: Tensor, gamma: Tensor, split: bool):
        zn = lazy_workspace_update(z, dz, gamma)
        ctx.save_for_backward(dz, gamma)
        ctx.z_dtype = z.dtype
        ctx.split = split
        ctx.set_materialize_grads(False)  # an unused Z_{l+1} (the last step's) skips the recurrence backward
        if split:
            return zn, zn.view_as(zn), dz.view_as(dz)
        return zn, dz.view_as(dz)

    @staticmethod
    def backward(ctx, *grads):
        grad_zn, grad_branch, grad_dz = grads if ctx.split else (grads[0], None, grads[1])
        dz, gamma = ctx.saved_tensors
        need = ctx.needs_input_grad
        if grad_zn is None:
            grad_zn, grad_branch = grad_branch, None
        if grad_zn is None:
            return None, grad_dz, None, None
        gdz = gg = None
        add = grad_dz if need[1] else None
        if grad_branch is not None:
            grad_zn, gdz, gg = lazy_workspace_update_backward_sum(grad_zn, grad_branch, dz, gamma, add)
        elif need[1] or need[2]:
            gdz, gg = lazy_workspace_update_backward(grad_zn, dz, gamma, add)
        grad_z = grad_zn.to(ctx.z_dtype) if need[0] else None
        gdz = gdz.to(dz.dtype) if need[1] and gdz is not None else None
        gg = gg.to(gamma.dtype) if need[2] and gg is not None else None
        return grad_z, gdz, gg, None


def lazy_workspace_step(z: Tensor, dz: Tensor, gamma: Tensor, split: bool = False) -> tuple[Tensor, ...]:
    """(lazy_workspace_update(z, dz, gamma), dz) with a fused backward for a later consumer of dz.

    Values are those of the separate uses; the backward of dz is gamma * g_next plus the later
    consumer's gradient, written by one recurrence-backward launch instead of a launch and an add.
    split=True returns (z_next, z_next for the branch, dz): the same values, with z_next's two
    gradients (next step, branch) summed by that launch too.
    """
    return _RecurStep.apply(z, dz, gamma, split)


# ---------------------------------------------------------------------------
# GAMMA STACK  gamma[l,c] = sum_k alpha[c,k] beta_stack[l,c,k]  (fp32)
# ---------------------------------------------------------------------------
@torch.library.custom_op("jit_thc::lazy_gamma_stack", mutates_args=())
def lazy_gamma_stack(alpha: Tensor, beta_stack: Tensor) -> Tensor:
    """fp32 [L,C] of gamma_l = sum_k alpha * beta_l (LayerLocalWrite.gamma_from_alpha for all layers)."""
    _on_gpu(alpha, beta_stack)
    if alpha.dim() != 2 or beta_stack.dim() != 3 or tuple(beta_stack.shape[1:]) != tuple(alpha.shape):
        raise ValueError(f"alpha [C,K] and beta_stack [L,C,K] expected, got {tuple(alpha.shape)}, {tuple(beta_stack.shape)}")
    L = beta_stack.shape[0]
    if not 1 <= L <= _abi.MAX_LAYERS:
        raise ValueError(f"depth {L} outside 1..{_abi.MAX_LAYERS}")
    (beta_stack,) = _same_dtype(alpha, [beta_stack])
    alpha, beta_stack = alpha.contiguous(), beta_stack.contiguous()
    c, k = alpha.shape
    out = torch.empty((L, c), device=alpha.device, dtype=torch.float32)
    with _on_device(alpha):
        rc = _abi.load().lthc_gamma(
            alpha.data_ptr(), _abi.ptr_array(list(beta_stack.unbind(0))), _abi.code(alpha), out.data_ptr(),
            _abi.F32, c, k, L, _abi.stream_of(alpha),
        )  # fmt: skip
    _abi.check(rc, "lthc_gamma")
    return out


@_fake(lazy_gamma_stack)
def _(alpha: Tensor, beta_stack: Tensor) -> Tensor:
    return alpha.new_empty((beta_stack.shape[0], alpha.shape[0]), dtype=torch.float32)


def _setup_gamma_ctx(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _backward_gamma(ctx, grad):
    alpha, beta_stack = ctx.saved_tensors
    g = grad.float()
    grad_alpha = (g[:, :, None] * beta_stack.float()).sum(0).to(alpha.dtype) if ctx.needs_input_grad[0] else None
    grad_beta = (g[:, :, None] * alpha.float()[None]).to(beta_stack.dtype) if ctx.needs_input_grad[1] else None
    return grad_alpha, grad_beta


torch.library.register_autograd(lazy_gamma_stack, _backward_gamma, setup_context=_setup_gamma_ctx)


# ---------------------------------------------------------------------------
# GAMMA OF EVERY LAYER WITH THE EAGER DTYPE SEQUENCE (one launch for the block hooks' gamma_from_alpha)
# ---------------------------------------------------------------------------
def lazy_gamma_rounded_eager(alpha: Tensor, betas: Sequence[Tensor], dtype: torch.dtype) -> Tensor:
    """[L, C] of (alpha.to(dtype) * beta_l.to(dtype)).sum(-1): gamma_from_alpha (local_thc.py:1278-1283) for each
    layer, alpha being the shared read's softmax cast to the workspace dtype (:1326)."""
    a = alpha.to(dtype)
    return torch.stack([(a * b.to(dtype)).sum(dim=-1) for b in betas])


@torch.library.custom_op("jit_thc::lazy_gamma_rounded", mutates_args=())
def lazy_gamma_rounded(alpha: Tensor, betas: list[Tensor], dtype: torch.dtype) -> Tensor:
    """[L, C] in `dtype` of r(sum_k r(r(alpha) r(beta_l))), r = round to `dtype`, the sum in fp32: the block hooks'
    gamma_from_alpha(shared_read.alpha(dtype)) for all layers in one launch."""
    _on_gpu(alpha, *betas)
    if alpha.dim() != 2 or not betas or any(tuple(b.shape) != tuple(alpha.shape) for b in betas):
        raise ValueError(f"alpha [C,K] and L betas of the same shape expected, got {tuple(alpha.shape)}")
    if not 1 <= len(betas) <= _abi.MAX_LAYERS:
        raise ValueError(f"depth {len(betas)} outside 1..{_abi.MAX_LAYERS}")
    bd = betas[0].dtype
    betas = [b.contiguous() if b.dtype == bd else b.to(bd).contiguous() for b in betas]
    alpha = alpha.contiguous()
    c, k = alpha.shape
    out = torch.empty((len(betas), c), device=alpha.device, dtype=dtype)
    with _on_device(alpha):
        rc = _abi.load().lthc_gamma_rounded(
            alpha.data_ptr(), _abi.code(alpha), _abi.ptr_array(betas), _abi.code(betas[0]), out.data_ptr(),
            _abi.code(out), c, k, len(betas), _abi.stream_of(alpha),
        )  # fmt: skip
    _abi.check(rc, "lthc_gamma_rounded")
    return out


@_fake(lazy_gamma_rounded)
def _(alpha: Tensor, betas: list[Tensor], dtype: torch.dtype) -> Tensor:
    return alpha.new_empty((len(betas), alpha.shape[0]), dtype=dtype)


def _setup_gamma_rounded_ctx(ctx, inputs, output):
    alpha, betas, dtype = inputs
    ctx.save_for_backward(alpha, *betas)
    ctx.dtype = dtype


@torch.library.custom_op("jit_thc::lazy_gamma_rounded_backward", mutates_args=())
def lazy_gamma_rounded_backward(
    grad: Tensor, alpha: Tensor, betas: list[Tensor], need_alpha: bool, need_beta: bool
) -> tuple[Tensor, list[Tensor]]:
    """Eager autograd's values for lazy_gamma_rounded_eager from one lthc_gamma_rounded_bwd launch: (grad of
    alpha, or an empty tensor when not needed; grads of the betas in the first beta's dtype, or an empty list).
    An op of its own so that the backward is opaque to torch.compile's tracing."""
    _on_gpu(grad, alpha, *betas)
    bd = betas[0].dtype
    betas = [b.contiguous() if b.dtype == bd else b.to(bd).contiguous() for b in betas]
    alpha = alpha.contiguous()
    grad = grad.contiguous()
    ga = torch.empty_like(alpha) if need_alpha else None
    gbs = [torch.empty_like(b) for b in betas] if need_beta else None
    c, k = alpha.shape
    with _on_device(alpha):
        rc = _abi.load().lthc_gamma_rounded_bwd(
            grad.data_ptr(), alpha.data_ptr(), _abi.code(alpha), _abi.ptr_array(betas), _abi.code(betas[0]),
            _abi.ptr(ga), _abi.ptr_array(gbs) if gbs is not None else None, _abi.code(grad), c, k, len(betas),
            _abi.stream_of(alpha),
        )  # fmt: skip
    _abi.check(rc, "lthc_gamma_rounded_bwd")
    return (ga if ga is not None else alpha.new_empty((0,))), (gbs if gbs is not None else [])


@_fake(lazy_gamma_rounded_backward)
def _(grad: Tensor, alpha: Tensor, betas: list[Tensor], need_alpha: bool, need_beta: bool):
    ga = alpha.new_empty(alpha.shape) if need_alpha else alpha.new_empty((0,))
    gbs = [betas[0].new_empty(b.shape) for b in betas] if need_beta else []
    return ga, gbs


def _backward_gamma_rounded(ctx, grad):
    """Eager autograd's values for lazy_gamma_rounded_eager, from one lthc_gamma_rounded_bwd launch."""
    alpha, *betas = ctx.saved_tensors
    need_a, need_b = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    if not (need_a or need_b):
        return None, None, None
    ga, gbs = lazy_gamma_rounded_backward(grad.to(ctx.dtype), alpha, betas, bool(need_a), bool(need_b))
    gbs = [g if g.dtype == b.dtype else g.to(b.dtype) for g, b in zip(gbs, betas)] if need_b else None
    return (ga if need_a else None), gbs, None


torch.library.register_autograd(lazy_gamma_rounded, _backward_gamma_rounded, setup_context=_setup_gamma_rounded_ctx)


# ---------------------------------------------------------------------------
# FINAL-LAYER RMSNORM + MODULATE (no reference op: FinalLayerSharedAdaLN's
# norm_final + modulate, local_thc.py:870-873, is eager torch)
# ---------------------------------------------------------------------------
def _check_norm(x: Tensor, weight: Tensor, shift: Tensor, scale: Tensor) -> tuple[int, int, int]:
    if x.dim() != 3:
        raise ValueError(f"x must be [B,N,C], got {tuple(x.shape)}")
    b, n, c = x.shape
    if tuple(weight.shape) != (c,) or tuple(shift.shape) != (b, c) or tuple(scale.shape) != (b, c):
        raise ValueError(
            f"weight [{c}], shift and scale [{b},{c}] expected, got {tuple(weight.shape)}, "
            f"{tuple(shift.shape)}, {tuple(scale.shape)}"
        )
    if shift.dtype != x.dtype or scale.dtype != x.dtype:
        raise ValueError(f"shift and scale must have x's dtype {x.dtype}, got {shift.dtype}, {scale.dtype}")
    if c % 4 != 0 or c > 2048:
        raise ValueError(f"channels {c} must be a multiple of 4 and at most 2048")
    _abi.code(x)
    return b, n, c


def _mod_rows(*ts: Tensor, elems: int = 4) -> tuple[list[Tensor], int]:
    """Per-sample [B, C] vectors as (tensors, common row stride): strided rows of one buffer (chunks of the shared
    AdaLN vector) are used in place when their rows are contiguous, share a stride that is a multiple of `elems`
    and start `elems`-element aligned; otherwise each is made contiguous (stride C)."""
    c = ts[0].shape[1]
    ld = ts[0].stride(0)
    ok = all(
        t.stride(1) == 1 and t.stride(0) == ld and (t.data_ptr() // t.element_size()) % elems == 0 for t in ts
    ) and ld >= c and ld % elems == 0
    if ok:
        return list(ts), ld
    out = [t.contiguous() for t in ts]
    out = [t if (t.data_ptr() // t.element_size()) % elems == 0 else t.clone() for t in out]
    return out, c


def _norm_weight(weight: Tensor) -> Tensor:
    """The RMSNorm weight as passed to the kernels: fp32, bf16 or fp16, contiguous."""
    w = weight if weight.dtype in (torch.float32, torch.bfloat16, torch.float16) else weight.float()
    w = w.contiguous()
    return w if w.data_ptr() % (4 * w.element_size()) == 0 else w.clone()  # 4-element vector loads


@torch.library.custom_op("jit_thc::norm_modulate", mutates_args=())
def norm_modulate(x: Tensor, weight: Tensor, shift: Tensor, scale: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """(modulate(RMSNorm(x), shift, scale) in x.dtype, fp32 [B*N] inverse RMS) in one pass over x."""
    _on_gpu(x, weight, shift, scale)
    b, n, c = _check_norm(x, weight, shift, scale)
    x = _prep(x)
    (shift, scale), ld = _mod_rows(shift, scale)
    w = _norm_weight(weight)
    y = torch.empty_like(x)
    inv = torch.empty((b * n,), device=x.device, dtype=torch.float32)
    with _on_device(x):
        rc = _abi.load().lthc_norm_modulate_fwd(
            x.data_ptr(), _abi.code(x), w.data_ptr(), _abi.code(w), shift.data_ptr(), scale.data_ptr(), ld,
            y.data_ptr(), inv.data_ptr(), b, n, c, eps, _abi.stream_of(x),
        )  # fmt: skip
    _abi.check(rc, "lthc_norm_modulate_fwd")
    return y, inv


@_fake(norm_modulate)
def _(x: Tensor, weight: Tensor, shift: Tensor, scale: Tensor, eps: float):
    return torch.empty_like(x), x.new_empty((x.shape[0] * x.shape[1],), dtype=torch.float32)


@torch.library.custom_op("jit_thc::norm_modulate_backward", mutates_args=())
def norm_modulate_backward(
    grad: Tensor, x: Tensor, weight: Tensor, scale: Tensor, inv: Tensor
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(dx in x.dtype, dweight fp32 [C], dshift fp32 [B,C], dscale fp32 [B,C])."""
    _on_gpu(grad, x, weight, scale, inv)
    b, n, c = _check_norm(x, weight, scale, scale)
    (grad,) = _same_dtype(x, [_prep(grad)])
    x, inv = _prep(x), inv.float().contiguous()
    (scale,), ld = _mod_rows(scale)
    w = _norm_weight(weight)
    gx = torch.empty_like(x)
    gw = torch.empty((c,), device=x.device, dtype=torch.float32)
    gsh = torch.empty((b, c), device=x.device, dtype=torch.float32)
    gsc = torch.empty((b, c), device=x.device, dtype=torch.float32)
    ws = torch.empty((max(_abi.norm_modulate_bwd_workspace_bytes(b, n, c), 16),), device=x.device, dtype=torch.uint8)
    with _on_device(x):
        rc = _abi.load().lthc_norm_modulate_bwd(
            grad.data_ptr(), x.data_ptr(), _abi.code(x), w.data_ptr(), _abi.code(w), scale.data_ptr(), ld,
            inv.data_ptr(), gx.data_ptr(), gw.data_ptr(), gsh.data_ptr(), gsc.data_ptr(), b, n, c, ws.data_ptr(),
            ws.numel(), _abi.stream_of(x),
        )  # fmt: skip
    _abi.check(rc, "lthc_norm_modulate_bwd")
    return gx, gw, gsh, gsc


@_fake(norm_modulate_backward)
def _(grad: Tensor, x: Tensor, weight: Tensor, scale: Tensor, inv: Tensor):
    b, n, c = x.shape
    f32 = torch.float32
    return torch.empty_like(x), x.new_empty((c,), dtype=f32), x.new_empty((b, c), dtype=f32), x.new_empty((b, c), dtype=f32)


def _setup_norm_ctx(ctx, inputs, output):
    x, weight, shift, scale, _ = inputs
    ctx.save_for_backward(x, weight, scale, output[1])
    ctx.dtypes = (weight.dtype, shift.dtype, scale.dtype)


def _backward_norm(ctx, grad_y, grad_inv):
    x, weight, scale, inv = ctx.saved_tensors
    gx, gw, gsh, gsc = norm_modulate_backward(grad_y.contiguous(), x, weight, scale, inv)
    wd, shd, scd = ctx.dtypes
    return gx, gw.to(wd), gsh.to(shd), gsc.to(scd), None


torch.library.register_autograd(norm_modulate, _backward_norm, setup_context=_setup_norm_ctx)


# ---------------------------------------------------------------------------
# DECODER HEAD: RMSNorm + modulate + linear + unpatchify in one pass (no reference op:
# FinalLayerSharedAdaLN.forward and unpatchify, local_thc.py:865-873 and :972-980, are eager torch)
# ---------------------------------------------------------------------------
DECODER_OUTPUTS = 48
DECODER_MAX_CHANNELS = 768


def decoder_head_supported(x: Tensor, lin_weight: Tensor) -> bool:
    """Whether jit_thc::decoder_head takes x [B, T, C]: 16-bit, C a multiple of 32 up to 768, T a multiple of 64,
    48 outputs per token."""
    return (
        x.is_cuda
        and x.dim() == 3
        and x.dtype in (torch.bfloat16, torch.float16)
        and x.shape[2] % 32 == 0
        and x.shape[2] <= DECODER_MAX_CHANNELS
        and x.shape[1] % 64 == 0
        and tuple(lin_weight.shape) == (DECODER_OUTPUTS, x.shape[2])
    )


def decoder_head_eager(x, norm_weight, shift, scale, lin_weight, lin_bias, eps: float, h: int, patch: int) -> Tensor:
    """The eager sequence: modulate(RMSNorm(x)) in x.dtype, the linear layer with its weight and bias cast to
    x.dtype (as autocast casts them), then unpatchify [B, h*w, P*P*CO] -> [B, CO, h*P, w*P]."""
    xf = x.float()
    n = (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps) * norm_weight).to(x.dtype)
    y = n * (1 + scale.unsqueeze(1)) + shift.unsqueeze(1)
    o = torch.nn.functional.linear(y, lin_weight.to(x.dtype), lin_bias.to(x.dtype))
    b, t, _ = x.shape
    w = t // h
    co = o.shape[-1] // (patch * patch)
    o = o.reshape(b, h, w, patch, patch, co).permute(0, 5, 1, 3, 2, 4)
    return o.reshape(b, co, h * patch, w * patch)


@torch.library.custom_op("jit_thc::decoder_head", mutates_args=())
def decoder_head(
    x: Tensor, norm_weight: Tensor, shift: Tensor, scale: Tensor, lin_weight: Tensor, lin_bias: Tensor, eps: float,
    h: int, patch: int,
) -> Tensor:
    """unpatchify(Linear(modulate(RMSNorm(x), shift, scale))) for x [B, h*w, C] (bf16 / fp16): the image
    [B, CO, h*P, w*P] in x.dtype, one pass over x (y stays in registers; the 48-output product on the matrix
    cores)."""
    _on_gpu(x, norm_weight, shift, scale, lin_weight, lin_bias)
    if not decoder_head_supported(x, lin_weight):
        raise ValueError(
            f"x must be bf16 or fp16 [B, T, C] with T % 64 == 0, C % 32 == 0, C <= {DECODER_MAX_CHANNELS} and "
            f"lin_weight [{DECODER_OUTPUTS}, C]; got {tuple(x.shape)} {x.dtype}, {tuple(lin_weight.shape)}"
        )
    b, t, c = x.shape
    if h <= 0 or t % h != 0 or patch != 4:
        raise ValueError(f"token grid {h} x {t // max(h, 1)} and patch {patch}: {t} tokens and 4 x 4 patches expected")
    w = t // h
    co = DECODER_OUTPUTS // (patch * patch)
    for name, v in (("shift", shift), ("scale", scale)):
        if tuple(v.shape) != (b, c) or v.dtype != x.dtype:
            raise ValueError(f"{name} must be [{b}, {c}] {x.dtype}, got {tuple(v.shape)} {v.dtype}")
    if tuple(norm_weight.shape) != (c,) or tuple(lin_bias.shape) != (DECODER_OUTPUTS,):
        raise ValueError(f"norm_weight [{c}] and lin_bias [{DECODER_OUTPUTS}] expected")
    x = _prep(x)
    (shift, scale), ld = _mod_rows(shift, scale, elems=1)
    nw = _norm_weight(norm_weight)
    lw = lin_weight if lin_weight.dtype in (torch.float32, x.dtype) else lin_weight.float()
    lb = lin_bias if lin_bias.dtype in (torch.float32, x.dtype) else lin_bias.float()
    lw, lb = lw.contiguous(), lb.contiguous()
    if lw.data_ptr() % 16 != 0:
        lw = lw.clone()
    img = torch.empty((b, co, h * patch, w * patch), device=x.device, dtype=x.dtype)
    with _on_device(x):
        rc = _abi.load().lthc_decoder_fwd(
            x.data_ptr(), _abi.code(x), nw.data_ptr(), _abi.code(nw), shift.data_ptr(), scale.data_ptr(), ld,
            lw.data_ptr(), _abi.code(lw), lb.data_ptr(), _abi.code(lb), img.data_ptr(), b, h, w, c, patch, co, eps,
            _abi.stream_of(x),
        )  # fmt: skip
    _abi.check(rc, "lthc_decoder_fwd")
    return img


def materialise_decoder_supported(x0: Tensor, dzs: Sequence[Tensor], lin_weight: Tensor, patch: int) -> bool:
    """Whether jit_thc::final_accumulate_decoder_head takes these operands: bf16 / fp16 x0 [B, 4G, 4G, C] with
    G % 16 == 0, C % 256 == 0, 1..12 layers, 4 x 4 patches of 3 channels (48 outputs per token), below 4 GiB."""
    if not (x0.is_cuda and x0.dim() == 4 and x0.dtype in (torch.bfloat16, torch.float16)):
        return False
    b, h, w, c = x0.shape
    return (
        h == w
        and h % (4 * 16) == 0
        and c % 256 == 0
        and 1 <= len(dzs) <= 12
        and patch == 4
        and tuple(lin_weight.shape) == (DECODER_OUTPUTS, c)
        and x0.numel() * 2 < 2**32
    )


@torch.library.custom_op("jit_thc::final_accumulate_decoder_head", mutates_args=())
def final_accumulate_decoder_head(
    x0: Tensor, dzs: list[Tensor], betas: list[Tensor], norm_weight: Tensor, shift: Tensor, scale: Tensor,
    lin_weight: Tensor, lin_bias: Tensor, eps: float, patch: int,
) -> Tensor:
    """The model's last two steps for no-grad forwards: X_L = x0 + sum_l P_l(dzs[l]) (local_thc.py:1368-1372)
    and unpatchify(Linear(modulate(RMSNorm(X_L), shift, scale))) (:865-873, :972-980), with X_L formed per token in
    registers and never written (lthc_materialise_decoder_fwd).  X_L is rounded to x0.dtype as the materialisation
    rounds it; the norm, modulation and linear layer are computed as inv * (x . M_b) + Q_b in fp32 without the
    eager sequence's intermediate roundings.  Returns the image [B, CO, 4G*P, 4G*P] in x0.dtype.  Inference only:
    no autograd formula."""
    _on_gpu(x0, *dzs, *betas, norm_weight, shift, scale, lin_weight, lin_bias)
    _check_list(x0, dzs, betas)
    if not materialise_decoder_supported(x0, dzs, lin_weight, patch):
        raise ValueError(
            f"x0 must be bf16 or fp16 [B, 4G, 4G, C] with G % 16 == 0, C % 256 == 0, 1..12 layers, lin_weight "
            f"[{DECODER_OUTPUTS}, C] and patch 4; got {tuple(x0.shape)} {x0.dtype}, {len(dzs)} layers, "
            f"{tuple(lin_weight.shape)}, patch {patch}"
        )
    b, h, _, c = x0.shape
    g = h // S
    co = DECODER_OUTPUTS // (patch * patch)
    for name, v in (("shift", shift), ("scale", scale)):
        if tuple(v.shape) != (b, c) or v.dtype != x0.dtype:
            raise ValueError(f"{name} must be [{b}, {c}] {x0.dtype}, got {tuple(v.shape)} {v.dtype}")
    if tuple(norm_weight.shape) != (c,) or tuple(lin_bias.shape) != (DECODER_OUTPUTS,):
        raise ValueError(f"norm_weight [{c}] and lin_bias [{DECODER_OUTPUTS}] expected")
    x0 = _prep(x0)
    dzs = _same_dtype(x0, [_prep(d) for d in dzs])
    betas = [_prep_w(bt, torch.float32).float() for bt in betas]
    (shift, scale), ld = _mod_rows(shift, scale, elems=1)
    nw = _norm_weight(norm_weight)
    lw = (lin_weight if lin_weight.dtype in (torch.float32, x0.dtype) else lin_weight.float()).contiguous()
    lb = (lin_bias if lin_bias.dtype in (torch.float32, x0.dtype) else lin_bias.float()).contiguous()
    img = torch.empty((b, co, h * patch, h * patch), device=x0.device, dtype=x0.dtype)
    ws = torch.empty((max(_abi.materialise_decoder_workspace_bytes(b, g, S, c), 16),), device=x0.device, dtype=torch.uint8)
    with _on_device(x0):
        rc = _abi.load().lthc_materialise_decoder_fwd(
            x0.data_ptr(), _abi.code(x0), _abi.ptr_array(dzs), _abi.ptr_array(betas), _abi.code(betas[0]),
            nw.data_ptr(), _abi.code(nw), shift.data_ptr(), scale.data_ptr(), ld, lw.data_ptr(), _abi.code(lw),
            lb.data_ptr(), _abi.code(lb), img.data_ptr(), b, g, S, c, len(dzs), patch, co, eps, ws.data_ptr(),
            ws.numel(), _abi.stream_of(x0),
        )  # fmt: skip
    _abi.check(rc, "lthc_materialise_decoder_fwd")
    return img


@_fake(final_accumulate_decoder_head)
def _(x0, dzs, betas, norm_weight, shift, scale, lin_weight, lin_bias, eps, patch):
    b, h, _, _ = x0.shape
    return x0.new_empty((b, DECODER_OUTPUTS // (patch * patch), h * patch, h * patch))


@_fake(decoder_head)
def _(x, norm_weight, shift, scale, lin_weight, lin_bias, eps, h, patch):
    b, t, _ = x.shape
    co = DECODER_OUTPUTS // (patch * patch)
    return x.new_empty((b, co, h * patch, (t // h) * patch))


def _setup_decoder_ctx(ctx, inputs, output):
    ctx.save_for_backward(*inputs[:6])
    ctx.geom = inputs[6:]


def _backward_decoder(ctx, grad):
    saved = ctx.saved_tensors
    need = ctx.needs_input_grad[:6]
    with torch.enable_grad():
        leaves = [t.detach().requires_grad_(bool(r)) for t, r in zip(saved, need)]
        out = decoder_head_eager(*leaves, *ctx.geom)
        wanted = [t for t in leaves if t.requires_grad]
        got = torch.autograd.grad([out], wanted, [grad], allow_unused=True) if wanted else []
    it = iter(got)
    return (*[next(it) if t.requires_grad else None for t in leaves], None, None, None)


torch.library.register_autograd(decoder_head, _backward_decoder, setup_context=_setup_decoder_ctx)


# ---------------------------------------------------------------------------
# BATCHED WEIGHT CONVERSION (autocast's per-forward weight casts in one launch)
# ---------------------------------------------------------------------------
_CAST_BLOCK = 2048  # elements per block of lthc_cast_many


class BatchedCast:
    """Converts a fixed list of contiguous fp32 tensors to `dtype` (round to nearest even, autocast's values) in
    one launch.  The outputs are views of one flat buffer, rewritten on every call; the conversion table is built
    once and holds the sources' addresses, so the sources are kept alive here and `key` identifies them."""

    def __init__(self, tensors: Sequence[Tensor], dtype: torch.dtype):
        if dtype not in (torch.bfloat16, torch.float16):
            raise ValueError(f"dtype must be bf16 or fp16, got {dtype}")
        if not tensors:
            raise ValueError("no tensors to convert")
        dev = tensors[0].device
        for t in tensors:
            if t.dtype != torch.float32 or not t.is_contiguous() or t.device != dev:
                raise ValueError("sources must be contiguous fp32 tensors on one device")
        self.key = (dtype, tuple((t.data_ptr(), t.numel()) for t in tensors))
        self.dtype = dtype
        self._src = list(tensors)
        entries, block_map, off, nblk = [], [], 0, 0
        for i, t in enumerate(tensors):
            n = t.numel()
            nb = (n + _CAST_BLOCK - 1) // _CAST_BLOCK
            entries.append((t.data_ptr(), n, off, nblk))
            block_map.extend([i] * nb)
            off += (n + 7) // 8 * 8
            nblk += nb
        self.nblocks = nblk
        self.buf = torch.empty((max(off, 8),), device=dev, dtype=dtype)
        self.entries = torch.tensor(entries, dtype=torch.int64).to(dev)
        self.block_map = torch.tensor(block_map, dtype=torch.int32).to(dev)
        self.outs = [self.buf[e[2]:e[2] + t.numel()].view(t.shape) for e, t in zip(entries, tensors)]

    def __call__(self) -> list[Tensor]:
        with _on_device(self.buf):
            rc = _abi.load().lthc_cast_many(
                self.entries.data_ptr(), self.block_map.data_ptr(), self.nblocks, self.buf.data_ptr(),
                _abi.code(self.buf), _abi.stream_of(self.buf),
            )  # fmt: skip
        _abi.check(rc, "lthc_cast_many")
        return self.outs


# Reference-style aliases (local_thc_triton_kernels.py exports these names).
triton_final_accumulate_b4_traceable = final_accumulate_b4_traceable
triton_final_accumulate_b4_12_traceable = final_accumulate_b4_12_traceable
