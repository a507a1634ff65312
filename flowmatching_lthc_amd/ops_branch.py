"""Fused elementwise ops of the LTHC transformer branch (gfx950 HIP kernels).

The reference evaluates these chains as eager PyTorch ops; they have no
``jit_thc`` counterpart there.  Each op here is one HIP pass with the eager
sequence's roundings (fp32 arithmetic, every eager op's result rounded to the
activation dtype), registered as a ``jit_thc`` custom op:

* ``jit_thc::qk_norm_rope``: ``rope(q_norm(q))`` and ``rope(k_norm(k))`` of
  ``WorkspaceAttention.forward`` (local_thc.py:246-249; RMSNorm
  jit_shared_adaln.py:26-30; VisionRotaryEmbeddingFast jit_shared_adaln.py:57-59),
  taking the qkv projection [B, N, 3, H, 64] and returning q and k as
  [B, N, H, 64] (the memory layout of the eager result);
* ``jit_thc::qk_norm_rope_attention``: the same q and k followed by
  ``F.scaled_dot_product_attention`` (local_thc.py:246-251), one matrix-core
  pass from the qkv projection to the attention output [B, N, H, 64];
* ``jit_thc::swiglu``: ``F.silu(x1) * x2`` of ``SwiGLUFFN.forward``
  (local_thc.py:267-269) for the w12 projection [..., 2F];
* ``jit_thc::gate_add_norm_modulate``: ``dz_attn = gate_msa * attn``,
  ``z_tmp = z + dz_attn`` and ``modulate(norm2(z_tmp), ...)`` of
  ``WorkspaceSharedAdaLNBranch.forward`` (local_thc.py:319-322);
* ``jit_thc::gate_residual``: its ``dz_attn + gate_mlp * mlp`` (:322-323);
* ``jit_thc::block_tail`` (inference): that gate_residual, the lazy
  recurrence step ``Z_{l+1} = Z_l + gamma_l * dZ_l`` (local_thc.py:1325-1328)
  and the next block's first pre-norm (:315-317) in one pass, each value
  that of the three separate ops.

The backward of all but gate_residual recomputes the eager sequence under
autograd (the forward's values are those of that sequence; the attention's
products accumulate in fp32 as SDPA's do), so training through them matches
the eager model's gradients; gate_residual's is its closed form.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor
from torch._subclasses.fake_tensor import is_fake

from . import _abi
from .ops import _fake, _mod_rows, _norm_weight, _on_device, _on_gpu

QK_HEAD_DIM = 64


# ---------------------------------------------------------------------------
# eager restatements (the backward recomputes these)
# ---------------------------------------------------------------------------
def _rms_norm_eager(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps) * weight).to(x.dtype)


def _rope_eager(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    pairs = x.unflatten(-1, (-1, 2))
    rot = torch.stack((-pairs[..., 1], pairs[..., 0]), dim=-1).flatten(-2)
    return x * cos.to(x.dtype) + rot * sin.to(x.dtype)


def qk_norm_rope_eager(qkv: Tensor, q_weight: Tensor, k_weight: Tensor, cos: Tensor, sin: Tensor, eps: float):
    """The eager sequence on qkv [B, N, 3, H, D]: (q, k) as [B, N, H, D] (cos / sin [N, D] broadcast over heads)."""
    c, s = cos[:, None, :], sin[:, None, :]
    q = _rope_eager(_rms_norm_eager(qkv[:, :, 0], q_weight, eps), c, s)
    k = _rope_eager(_rms_norm_eager(qkv[:, :, 1], k_weight, eps), c, s)
    return q, k


def swiglu_eager(x: Tensor) -> Tensor:
    a, v = x.chunk(2, dim=-1)
    return F.silu(a) * v


def _aligned(t: Tensor) -> Tensor:
    """Contiguous with a 16-byte aligned start (the kernels use 16-byte vector accesses)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


# ---------------------------------------------------------------------------
# jit_thc::qk_norm_rope
# ---------------------------------------------------------------------------
def _check_qk(qkv: Tensor, q_weight: Tensor, k_weight: Tensor, cos: Tensor, sin: Tensor) -> tuple[int, int, int]:
    if qkv.dim() != 5 or qkv.shape[2] != 3 or qkv.shape[4] != QK_HEAD_DIM:
        raise ValueError(f"qkv must be [B,N,3,H,{QK_HEAD_DIM}], got {tuple(qkv.shape)}")
    b, n, _, h, d = qkv.shape
    if tuple(q_weight.shape) != (d,) or tuple(k_weight.shape) != (d,):
        raise ValueError(f"q/k norm weights must be [{d}], got {tuple(q_weight.shape)}, {tuple(k_weight.shape)}")
    if tuple(cos.shape) != (n, d) or tuple(sin.shape) != (n, d):
        raise ValueError(f"RoPE tables must be [{n},{d}], got {tuple(cos.shape)}, {tuple(sin.shape)}")
    _abi.code(qkv)
    return b, n, h


@torch.library.custom_op("jit_thc::qk_norm_rope", mutates_args=())
def qk_norm_rope(qkv: Tensor, q_weight: Tensor, k_weight: Tensor, cos: Tensor, sin: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """(rope(RMSNorm_q(q)), rope(RMSNorm_k(k))) as [B, N, H, 64] in qkv's dtype, one pass over q and k."""
    _on_gpu(qkv, q_weight, k_weight, cos, sin)
    b, n, h = _check_qk(qkv, q_weight, k_weight, cos, sin)
    qkv = _aligned(qkv)
    # weights and tables: fp32 or the activation dtype (bf16 parameters and buffers are used as they are)
    qw, kw, c, s = (t if t.dtype == qkv.dtype else t.float() for t in (q_weight, k_weight, cos, sin))
    if kw.dtype != qw.dtype:
        qw, kw = qw.float(), kw.float()
    if s.dtype != c.dtype:
        c, s = c.float(), s.float()
    qw, kw, c, s = (_aligned(t) for t in (qw, kw, c, s))
    q = torch.empty((b, n, h, QK_HEAD_DIM), device=qkv.device, dtype=qkv.dtype)
    k = torch.empty_like(q)
    with _on_device(qkv):
        rc = _abi.load().lthc_qk_norm_rope(
            qkv.data_ptr(), _abi.code(qkv), qw.data_ptr(), kw.data_ptr(), _abi.code(qw), c.data_ptr(), s.data_ptr(),
            _abi.code(c), q.data_ptr(), k.data_ptr(), b, n, h, QK_HEAD_DIM, eps, _abi.stream_of(qkv),
        )  # fmt: skip
    _abi.check(rc, "lthc_qk_norm_rope")
    return q, k


@_fake(qk_norm_rope)
def _(qkv, q_weight, k_weight, cos, sin, eps):
    b, n, _, h, d = qkv.shape
    return qkv.new_empty((b, n, h, d)), qkv.new_empty((b, n, h, d))


def _setup_qk_ctx(ctx, inputs, output):
    qkv, q_weight, k_weight, cos, sin, eps = inputs
    ctx.save_for_backward(qkv, q_weight, k_weight, cos, sin)
    ctx.eps = eps


def _backward_qk(ctx, grad_q, grad_k):
    qkv, q_weight, k_weight, cos, sin = ctx.saved_tensors
    need = ctx.needs_input_grad
    with torch.enable_grad():
        leaves = [t.detach().requires_grad_(bool(r)) for t, r in zip((qkv, q_weight, k_weight), need[:3])]
        q, k = qk_norm_rope_eager(leaves[0], leaves[1], leaves[2], cos, sin, ctx.eps)
        outs, grads = [], []
        for o, g in ((q, grad_q), (k, grad_k)):
            if g is not None:
                outs.append(o)
                grads.append(g)
        wanted = [t for t in leaves if t.requires_grad]
        got = torch.autograd.grad(outs, wanted, grads, allow_unused=True) if outs and wanted else []
    it = iter(got)
    res = [next(it) if t.requires_grad else None for t in leaves]
    return res[0], res[1], res[2], None, None, None


torch.library.register_autograd(qk_norm_rope, _backward_qk, setup_context=_setup_qk_ctx)


# ---------------------------------------------------------------------------
# jit_thc::qk_norm_rope_attention
# ---------------------------------------------------------------------------
ATTN_MAX_TOKENS = 256


def attention_supported(qkv: Tensor) -> bool:
    """Whether jit_thc::qk_norm_rope_attention takes qkv [B, N, 3, H, 64]: 16-bit, N a multiple of 64 up to 256."""
    n = qkv.shape[1]
    return (
        qkv.is_cuda
        and qkv.dtype in (torch.bfloat16, torch.float16)
        and qkv.dim() == 5
        and qkv.shape[4] == QK_HEAD_DIM
        and n % 64 == 0
        and 0 < n <= ATTN_MAX_TOKENS
    )


def qk_norm_rope_attention_eager(qkv: Tensor, q_weight: Tensor, k_weight: Tensor, cos: Tensor, sin: Tensor, eps: float):
    """q/k norm + RoPE, then F.scaled_dot_product_attention (default scale, no mask): o as [B, N, H, D]."""
    q, k = qk_norm_rope_eager(qkv, q_weight, k_weight, cos, sin, eps)
    v = qkv[:, :, 2]
    # [B, H, N, D] operands made contiguous (no transposed views in the batched products)
    q, k, v = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    o = F.scaled_dot_product_attention(q, k, v)
    return o.transpose(1, 2)


@torch.library.custom_op("jit_thc::qk_norm_rope_attention", mutates_args=())
def qk_norm_rope_attention(qkv: Tensor, q_weight: Tensor, k_weight: Tensor, cos: Tensor, sin: Tensor, eps: float) -> Tensor:
    """softmax(q_n k_n^T / sqrt(64)) v for q_n, k_n = qk_norm_rope(...): o as [B, N, H, 64] in qkv's dtype (bf16 or
    fp16, N a multiple of 64 up to 256), one pass over qkv on the matrix cores."""
    _on_gpu(qkv, q_weight, k_weight, cos, sin)
    b, n, h = _check_qk(qkv, q_weight, k_weight, cos, sin)
    if not attention_supported(qkv):
        raise ValueError(f"qkv must be bf16 or fp16 [B,N,3,H,64] with N a multiple of 64 up to {ATTN_MAX_TOKENS}, got "
                         f"{tuple(qkv.shape)} {qkv.dtype}")
    qkv = _aligned(qkv)
    qw, kw, c, s = (t if t.dtype == qkv.dtype else t.float() for t in (q_weight, k_weight, cos, sin))
    if kw.dtype != qw.dtype:
        qw, kw = qw.float(), kw.float()
    if s.dtype != c.dtype:
        c, s = c.float(), s.float()
    qw, kw, c, s = (_aligned(t) for t in (qw, kw, c, s))
    out = torch.empty((b, n, h, QK_HEAD_DIM), device=qkv.device, dtype=qkv.dtype)
    with _on_device(qkv):
        rc = _abi.load().lthc_qk_norm_rope_attention(
            qkv.data_ptr(), _abi.code(qkv), qw.data_ptr(), kw.data_ptr(), _abi.code(qw), c.data_ptr(), s.data_ptr(),
            _abi.code(c), out.data_ptr(), b, n, h, QK_HEAD_DIM, eps, QK_HEAD_DIM**-0.5, _abi.stream_of(qkv),
        )  # fmt: skip
    _abi.check(rc, "lthc_qk_norm_rope_attention")
    return out


@_fake(qk_norm_rope_attention)
def _(qkv, q_weight, k_weight, cos, sin, eps):
    b, n, _, h, d = qkv.shape
    return qkv.new_empty((b, n, h, d))


def _attention_fp32_recompute(qkv: Tensor, q_weight: Tensor, k_weight: Tensor, cos: Tensor, sin: Tensor, eps: float):
    """qk_norm_rope_attention_eager's function with the attention itself in fp32 matrix products and softmax
    (softmax(q k^T / sqrt(64)) v, rounded once to qkv's dtype): the backward's recompute when torch.compile traces it.
    Plain products, not the SDPA kernels: the ROCm flash-attention backward returns gradient strides its meta function
    does not predict, which compiled graphs assert on.  Eager backwards keep the SDPA recompute (at B=64 the fp32
    products made the LTHC-B/4 training step 25 % slower)."""
    q, k = qk_norm_rope_eager(qkv, q_weight, k_weight, cos, sin, eps)
    v = qkv[:, :, 2]
    q, k, v = (t.transpose(1, 2).float().contiguous() for t in (q, k, v))
    kt = k.transpose(-1, -2).contiguous()
    p = torch.softmax(torch.matmul(q, kt) * (QK_HEAD_DIM**-0.5), dim=-1)
    return torch.matmul(p, v).to(qkv.dtype).transpose(1, 2)


def _traced(t: Tensor) -> bool:
    """True while torch.compile traces the code (Dynamo, or AOTAutograd on fake tensors), False when it runs."""
    return torch.compiler.is_compiling() or is_fake(t)


def _backward_qk_attention(ctx, grad):
    qkv, q_weight, k_weight, cos, sin = ctx.saved_tensors
    need = ctx.needs_input_grad
    # eager: the SDPA recompute (flash / efficient kernels); traced: fp32 products, whose strides the graph predicts
    recompute = _attention_fp32_recompute if _traced(grad) else qk_norm_rope_attention_eager
    with torch.enable_grad():
        leaves = [t.detach().requires_grad_(bool(r)) for t, r in zip((qkv, q_weight, k_weight), need[:3])]
        o = recompute(leaves[0], leaves[1], leaves[2], cos, sin, ctx.eps)
        wanted = [t for t in leaves if t.requires_grad]
        got = torch.autograd.grad([o], wanted, [grad], allow_unused=True) if wanted else []
    it = iter(got)
    res = [next(it) if t.requires_grad else None for t in leaves]
    return res[0], res[1], res[2], None, None, None


torch.library.register_autograd(qk_norm_rope_attention, _backward_qk_attention, setup_context=_setup_qk_ctx)


# ---------------------------------------------------------------------------
# jit_thc::swiglu
# ---------------------------------------------------------------------------
@torch.library.custom_op("jit_thc::swiglu", mutates_args=())
def swiglu(x: Tensor) -> Tensor:
    """silu(x[..., :F]) * x[..., F:] in x's dtype for x [..., 2F], F % 8 == 0."""
    _on_gpu(x)
    two_f = x.shape[-1]
    if two_f % 16 != 0:
        raise ValueError(f"last dimension {two_f} must be 2F with F a multiple of 8")
    f = two_f // 2
    _abi.code(x)
    x = _aligned(x)
    out = torch.empty((*x.shape[:-1], f), device=x.device, dtype=x.dtype)
    rows = x.numel() // two_f
    with _on_device(x):
        rc = _abi.load().lthc_swiglu(x.data_ptr(), _abi.code(x), out.data_ptr(), rows, f, _abi.stream_of(x))
    _abi.check(rc, "lthc_swiglu")
    return out


@_fake(swiglu)
def _(x):
    return x.new_empty((*x.shape[:-1], x.shape[-1] // 2))


def _setup_swiglu_ctx(ctx, inputs, output):
    ctx.save_for_backward(inputs[0])


def _backward_swiglu(ctx, grad):
    (x,) = ctx.saved_tensors
    with torch.enable_grad():
        xl = x.detach().requires_grad_()
        (gx,) = torch.autograd.grad(swiglu_eager(xl), (xl,), (grad,))
    return gx


torch.library.register_autograd(swiglu, _backward_swiglu, setup_context=_setup_swiglu_ctx)


# ---------------------------------------------------------------------------
# gated residuals of the branch: jit_thc::gate_add_norm_modulate, jit_thc::gate_residual
# (WorkspaceSharedAdaLNBranch.forward, local_thc.py:319-323)
# ---------------------------------------------------------------------------
def gate_add_norm_modulate_eager(z: Tensor, a: Tensor, gate: Tensor, weight: Tensor, shift: Tensor, scale: Tensor, eps: float):
    """(d, y): d = gate * a, y = modulate(RMSNorm(z + d), shift, scale), as the eager branch evaluates them."""
    d = gate.unsqueeze(1) * a
    n = _rms_norm_eager(z + d, weight, eps)
    return d, n * (1 + scale.unsqueeze(1)) + shift.unsqueeze(1)


def gate_residual_eager(d: Tensor, gate: Tensor, m: Tensor) -> Tensor:
    return d + gate.unsqueeze(1) * m


def _check_bnc(name: str, t: Tensor, shape: tuple, dtype: torch.dtype) -> None:
    if tuple(t.shape) != shape or t.dtype != dtype:
        raise ValueError(f"{name} must be {list(shape)} {dtype}, got {tuple(t.shape)} {t.dtype}")


@torch.library.custom_op("jit_thc::gate_add_norm_modulate", mutates_args=())
def gate_add_norm_modulate(
    z: Tensor, a: Tensor, gate: Tensor, weight: Tensor, shift: Tensor, scale: Tensor, eps: float
) -> tuple[Tensor, Tensor]:
    """(gate * a, modulate(RMSNorm(z + gate * a), shift, scale)) in z's dtype, one pass; z, a [B,N,C], the rest [B,C]
    (weight [C])."""
    _on_gpu(z, a, gate, weight, shift, scale)
    if z.dim() != 3:
        raise ValueError(f"z must be [B,N,C], got {tuple(z.shape)}")
    b, n, c = z.shape
    _check_bnc("a", a, (b, n, c), z.dtype)
    for name, t in (("gate", gate), ("shift", shift), ("scale", scale)):
        _check_bnc(name, t, (b, c), z.dtype)
    if tuple(weight.shape) != (c,):
        raise ValueError(f"weight must be [{c}], got {tuple(weight.shape)}")
    _abi.code(z)
    z, a = _aligned(z), _aligned(a)
    (gate, shift, scale), ld = _mod_rows(gate, shift, scale)
    w = _norm_weight(weight)
    d, y = torch.empty_like(z), torch.empty_like(z)
    with _on_device(z):
        rc = _abi.load().lthc_gate_add_norm_modulate_fwd(
            z.data_ptr(), a.data_ptr(), gate.data_ptr(), _abi.code(z), w.data_ptr(), _abi.code(w), shift.data_ptr(),
            scale.data_ptr(), ld, d.data_ptr(), y.data_ptr(), None, b, n, c, eps, _abi.stream_of(z),
        )  # fmt: skip
    _abi.check(rc, "lthc_gate_add_norm_modulate_fwd")
    return d, y


@_fake(gate_add_norm_modulate)
def _(z, a, gate, weight, shift, scale, eps):
    return torch.empty_like(z), torch.empty_like(z)


def _setup_ganm_ctx(ctx, inputs, output):
    ctx.save_for_backward(*inputs[:6])
    ctx.eps = inputs[6]


def _backward_ganm(ctx, grad_d, grad_y):
    saved = ctx.saved_tensors
    need = ctx.needs_input_grad[:6]
    with torch.enable_grad():
        leaves = [t.detach().requires_grad_(bool(r)) for t, r in zip(saved, need)]
        d, y = gate_add_norm_modulate_eager(*leaves, ctx.eps)
        outs = [o for o, g in ((d, grad_d), (y, grad_y)) if g is not None]
        grads = [g for g in (grad_d, grad_y) if g is not None]
        wanted = [t for t in leaves if t.requires_grad]
        got = torch.autograd.grad(outs, wanted, grads, allow_unused=True) if outs and wanted else []
    it = iter(got)
    return (*[next(it) if t.requires_grad else None for t in leaves], None)


torch.library.register_autograd(gate_add_norm_modulate, _backward_ganm, setup_context=_setup_ganm_ctx)


@torch.library.custom_op("jit_thc::gate_residual", mutates_args=())
def gate_residual(d: Tensor, gate: Tensor, m: Tensor) -> Tensor:
    """d + gate * m in d's dtype for d, m [B,N,C] and a per-sample gate [B,C] (C % 8 == 0)."""
    _on_gpu(d, gate, m)
    if d.dim() != 3 or d.shape[2] % 8 != 0:
        raise ValueError(f"d must be [B,N,C] with C % 8 == 0, got {tuple(d.shape)}")
    b, n, c = d.shape
    _check_bnc("m", m, (b, n, c), d.dtype)
    _check_bnc("gate", gate, (b, c), d.dtype)
    _abi.code(d)
    d, m = _aligned(d), _aligned(m)
    (gate,), ld = _mod_rows(gate, elems=8)
    out = torch.empty_like(d)
    with _on_device(d):
        rc = _abi.load().lthc_gate_residual(
            d.data_ptr(), gate.data_ptr(), ld, m.data_ptr(), _abi.code(d), out.data_ptr(), b, n, c, _abi.stream_of(d)
        )
    _abi.check(rc, "lthc_gate_residual")
    return out


@_fake(gate_residual)
def _(d, gate, m):
    return torch.empty_like(d)


def _setup_gres_ctx(ctx, inputs, output):
    d, gate, m = inputs
    ctx.save_for_backward(gate, m)


def _backward_gres(ctx, grad):
    gate, m = ctx.saved_tensors
    need = ctx.needs_input_grad
    grad_d = grad if need[0] else None
    grad_gate = (grad * m).float().sum(1).to(gate.dtype) if need[1] else None
    grad_m = grad * gate.unsqueeze(1) if need[2] else None
    return grad_d, grad_gate, grad_m


torch.library.register_autograd(gate_residual, _backward_gres, setup_context=_setup_gres_ctx)


# ---------------------------------------------------------------------------
# block tail (inference): gate_residual + recurrence step + the next block's first pre-norm
# ---------------------------------------------------------------------------
@torch.library.custom_op("jit_thc::block_tail", mutates_args=())
def block_tail(
    z: Tensor, a: Tensor, gate: Tensor, m: Tensor, gamma: Tensor, weight: Tensor, shift: Tensor, scale: Tensor,
    eps: float,
) -> tuple[Tensor, Tensor, Tensor]:
    """(dz, z_next, y) = (a + gate * m, z + gamma * dz, modulate(RMSNorm(z_next), shift, scale)) in z's dtype, one
    pass: gate_residual, lazy_workspace_update and the next block's norm_modulate with the same values.  z, a, m
    [B,N,C]; gate, shift, scale [B,C]; gamma and weight [C].  Forward only (inference)."""
    _on_gpu(z, a, gate, m, gamma, weight, shift, scale)
    if z.dim() != 3 or z.shape[2] % 8 != 0:
        raise ValueError(f"z must be [B,N,C] with C % 8 == 0, got {tuple(z.shape)}")
    b, n, c = z.shape
    _check_bnc("a", a, (b, n, c), z.dtype)
    _check_bnc("m", m, (b, n, c), z.dtype)
    for name, t in (("gate", gate), ("shift", shift), ("scale", scale)):
        _check_bnc(name, t, (b, c), z.dtype)
    for name, t in (("gamma", gamma), ("weight", weight)):
        if tuple(t.shape) != (c,):
            raise ValueError(f"{name} must be [{c}], got {tuple(t.shape)}")
    _abi.code(z)
    z, a, m = _aligned(z), _aligned(a), _aligned(m)
    (gate, shift, scale), ld = _mod_rows(gate, shift, scale)
    w = _norm_weight(weight)
    g = _norm_weight(gamma)
    dz, zn, y = torch.empty_like(z), torch.empty_like(z), torch.empty_like(z)
    with _on_device(z):
        rc = _abi.load().lthc_block_tail_fwd(
            z.data_ptr(), a.data_ptr(), m.data_ptr(), gate.data_ptr(), _abi.code(z), g.data_ptr(), _abi.code(g),
            w.data_ptr(), _abi.code(w), shift.data_ptr(), scale.data_ptr(), ld, dz.data_ptr(), zn.data_ptr(),
            y.data_ptr(), b, n, c, eps, _abi.stream_of(z),
        )  # fmt: skip
    _abi.check(rc, "lthc_block_tail_fwd")
    return dz, zn, y


@_fake(block_tail)
def _(z, a, gate, m, gamma, weight, shift, scale, eps):
    return torch.empty_like(z), torch.empty_like(z), torch.empty_like(z)
