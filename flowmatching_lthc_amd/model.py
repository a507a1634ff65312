"""LTHC-B/4 shared-read model around the HIP interface.

The high-resolution interface -- shared read, lazy workspace recurrence and
the single final materialisation -- runs through the ``jit_thc`` HIP ops of
:mod:`.ops`.  The workspace transformer, embedders and decoder are PyTorch
modules whose GEMMs and attention run through hipBLASLt / the SDPA kernels of
PyTorch-ROCm; their elementwise chains (RMSNorm + modulate, q/k norm + RoPE,
SwiGLU, gated residuals) run through the fused HIP ops of :mod:`.ops` and
:mod:`.ops_branch` on the GPU, with the eager sequence as the reference and
the fallback for shapes those kernels do not take.

The module tree, parameter names, initialisation and forward math follow
flowmatching_lthc/models/local_thc.py (SharedReadLocalTHCSharedAdaLNJiT,
:1331-1394, its FusedFinal12 subclass :1413-1420 and the components at
:84-323, :853-1007) and flowmatching_lthc/models/jit_shared_adaln.py
(RMSNorm :20-30, VisionRotaryEmbeddingFast :33-59), so a reference state dict
loads unchanged and ``build_model('lthc_b4_velocity')`` builds the same network.
"""

from __future__ import annotations

import math
import re
from contextlib import contextmanager, nullcontext

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from . import ops, ops_branch
from .local_thc import LayerLocalWrite, SharedLocalRead, overridden


def modulate(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """x * (1 + scale) + shift with per-sample [B, C] shift/scale (local_thc.py:37-38)."""
    return x * (1 + scale.unsqueeze(1)) + shift.unsqueeze(1)


class CastLinear(nn.Linear):
    """nn.Linear that, while the model's forward has converted every weight in one batched launch
    (``BatchedWeightCast._converted_weights``), multiplies by that (weight, bias) pair: the values
    autocast's own per-layer conversion would give.  Parameters and state-dict names are nn.Linear's."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        cast = self.__dict__.get("_cast")
        if cast is not None:
            return F.linear(x, cast[0], cast[1])
        return super().forward(x)


class RMSNorm(nn.Module):
    """RMS normalisation computed in fp32, returned in the input dtype (jit_shared_adaln.py:20-30)."""

    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        inv = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return (xf * inv * self.weight).to(x.dtype)


def norm_modulate(norm: RMSNorm, x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """modulate(norm(x), shift, scale) for x [B, N, C] and per-sample [B, C] shift / scale.

    On the GPU, when shift and scale share x's dtype (bf16 autocast or fp32), one HIP pass with the eager
    sequence's roundings (jit_thc::norm_modulate); otherwise the eager sequence itself (other dtype mixes
    follow torch's promotion rules, which the kernel does not implement).
    """
    if x.is_cuda and x.dim() == 3 and shift.dtype == x.dtype and scale.dtype == x.dtype and x.shape[-1] % 4 == 0 and x.shape[-1] <= 2048:
        return ops.norm_modulate(x, norm.weight, shift, scale, norm.eps)[0]
    return modulate(norm(x), shift, scale)


def _rotate_pairs(x: torch.Tensor) -> torch.Tensor:
    """(x0, x1, x2, x3, ...) -> (-x1, x0, -x3, x2, ...): rotation of interleaved pairs."""
    pairs = x.unflatten(-1, (-1, 2))
    return torch.stack((-pairs[..., 1], pairs[..., 0]), dim=-1).flatten(-2)


class VisionRotaryEmbeddingFast(nn.Module):
    """2-D rotary embedding over a grid x grid token map (jit_shared_adaln.py:33-59).

    A head of 2*dim channels rotates its first dim channels with the token's
    row position and the last dim channels with its column position, in
    interleaved (even, odd) pairs.
    """

    def __init__(self, dim: int, grid_size: int, num_prefix_tokens: int = 0, theta: float = 10000.0) -> None:
        super().__init__()
        inv = 1.0 / (theta ** (torch.arange(0, dim, 2).float()[: dim // 2] / dim))
        pos = torch.arange(grid_size).float()
        ang = torch.outer(pos, inv).repeat_interleave(2, dim=-1)  # [grid, dim]
        rows = ang[:, None, :].expand(grid_size, grid_size, dim)
        cols = ang[None, :, :].expand(grid_size, grid_size, dim)
        table = torch.cat([rows, cols], dim=-1).reshape(grid_size * grid_size, 2 * dim)
        cos, sin = table.cos(), table.sin()
        if num_prefix_tokens:
            cos = torch.cat([torch.ones(num_prefix_tokens, cos.shape[-1]), cos], dim=0)
            sin = torch.cat([torch.zeros(num_prefix_tokens, sin.shape[-1]), sin], dim=0)
        self.register_buffer("freqs_cos", cos, persistent=False)
        self.register_buffer("freqs_sin", sin, persistent=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        cos = self.freqs_cos.to(x.device, x.dtype)
        sin = self.freqs_sin.to(x.device, x.dtype)
        return x * cos + _rotate_pairs(x) * sin

    def tables(self, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
        """(cos, sin) cast to `dtype` -- the values forward() multiplies by -- converted once and kept until the
        buffers change (a new device or dtype, or an in-place update)."""
        if self.freqs_cos.dtype == dtype:
            return self.freqs_cos, self.freqs_sin
        if torch.compiler.is_compiling():  # the compiled graph holds the conversion (no cache keyed on addresses)
            return self.freqs_cos.to(dtype), self.freqs_sin.to(dtype)
        key = (dtype, self.freqs_cos.data_ptr(), self.freqs_cos._version, self.freqs_sin.data_ptr(), self.freqs_sin._version)
        cache = self.__dict__.get("_cast_tables")
        if cache is None or cache[0] != key:
            cache = (key, self.freqs_cos.to(dtype), self.freqs_sin.to(dtype))
            self.__dict__["_cast_tables"] = cache
        return cache[1], cache[2]


def _patch_rows(x: torch.Tensor, p: int, grid: tuple[int, int]) -> torch.Tensor:
    """[B, Cin, H, W] -> [B, H/p, W/p, Cin*p*p]: each non-overlapping p x p patch as one row in (channel, row,
    column) order, the layout of a kernel = stride = p convolution's weight.  Under CUDA autocast an fp32 image is
    gathered and cast in one copy (the values autocast's cast of the gathered rows would give)."""
    b, cin = x.shape[:2]
    gh, gw = grid
    view = x.reshape(b, cin, gh, p, gw, p).permute(0, 2, 4, 1, 3, 5)
    if x.is_cuda and x.dtype == torch.float32 and torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
        return torch.empty((b, gh, gw, cin, p, p), device=x.device, dtype=dt).copy_(view).view(b, gh, gw, cin * p * p)
    return view.reshape(b, gh, gw, cin * p * p)


class BottleneckPatchEmbedNHWC(nn.Module):
    """Conv patchify (in -> bottleneck, kernel = stride = patch) then 1x1 conv to C, NHWC out (local_thc.py:64-89)."""

    def __init__(
        self,
        img_size: int = 256,
        patch_size: int = 4,
        in_chans: int = 3,
        bottleneck_dim: int = 128,
        embed_dim: int = 768,
        bias: bool = True,
    ) -> None:
        super().__init__()
        self.img_size = (img_size, img_size)
        self.patch_size = (patch_size, patch_size)
        self.grid_size = (img_size // patch_size, img_size // patch_size)
        self.num_patches = self.grid_size[0] * self.grid_size[1]
        self.proj1 = nn.Conv2d(in_chans, bottleneck_dim, kernel_size=patch_size, stride=patch_size, bias=False)
        self.proj2 = nn.Conv2d(bottleneck_dim, embed_dim, kernel_size=1, stride=1, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if tuple(x.shape[-2:]) != self.img_size:
            raise ValueError(f"expected image size {self.img_size}, got {tuple(x.shape[-2:])}")
        # proj1 has kernel = stride = patch and no bias: a linear map of each non-overlapping patch (channel,
        # row, column order, the layout of its weight).  proj2 is a 1x1 convolution: a linear map over proj1's
        # channels.  As two GEMMs over patch rows in NHWC order the residual comes out NHWC directly, with
        # proj2's bias in the GEMM (no permute copy of the C-channel tensor, no separate bias pass).
        patches = _patch_rows(x, self.patch_size[0], self.grid_size)
        cast = self.__dict__.get("_cast")
        w1, w2, b2 = cast if cast is not None else (self.proj1.weight, self.proj2.weight, self.proj2.bias)
        h = F.linear(patches, w1.view(self.proj1.out_channels, -1))
        return F.linear(h, w2.view(self.proj2.out_channels, -1), b2)

    def cast_targets(self) -> list[torch.Tensor] | None:
        """The tensors forward() takes, in order, from a batched conversion set as ``_cast`` (None: no such form)."""
        return [self.proj1.weight, self.proj2.weight, self.proj2.bias] if self.proj2.bias is not None else None


class DirectPatchEmbedNHWC(nn.Module):
    """One conv patchify (in -> C, kernel = stride = patch), NHWC out (local_thc.py:92-119), as one GEMM over the
    patch rows in NHWC order (the conv's weight is a linear map of each patch in channel, row, column order)."""

    def __init__(
        self,
        img_size: int = 256,
        patch_size: int = 4,
        in_chans: int = 3,
        bottleneck_dim: int = 128,
        embed_dim: int = 768,
        bias: bool = True,
    ) -> None:
        super().__init__()
        self.img_size = (img_size, img_size)
        self.patch_size = (patch_size, patch_size)
        self.grid_size = (img_size // patch_size, img_size // patch_size)
        self.num_patches = self.grid_size[0] * self.grid_size[1]
        self.proj = nn.Conv2d(in_chans, embed_dim, kernel_size=patch_size, stride=patch_size, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if tuple(x.shape[-2:]) != self.img_size:
            raise ValueError(f"expected image size {self.img_size}, got {tuple(x.shape[-2:])}")
        patches = _patch_rows(x, self.patch_size[0], self.grid_size)
        cast = self.__dict__.get("_cast")
        w, bias = cast if cast is not None else (self.proj.weight, self.proj.bias)
        return F.linear(patches, w.view(self.proj.out_channels, -1), bias)

    def cast_targets(self) -> list[torch.Tensor] | None:
        """The tensors forward() takes, in order, from a batched conversion set as ``_cast`` (None: no such form)."""
        return [self.proj.weight, self.proj.bias] if self.proj.bias is not None else None


class TimestepEmbedder(nn.Module):
    """Sinusoidal timestep features (cos then sin) through a 2-layer SiLU MLP (local_thc.py:175-200)."""

    def __init__(self, hidden_size: int, frequency_embedding_size: int = 256) -> None:
        super().__init__()
        self.frequency_embedding_size = frequency_embedding_size
        self.mlp = nn.Sequential(
            CastLinear(frequency_embedding_size, hidden_size, bias=True),
            nn.SiLU(),
            CastLinear(hidden_size, hidden_size, bias=True),
        )

    @staticmethod
    def timestep_embedding(t: torch.Tensor, dim: int, max_period: int = 10000) -> torch.Tensor:
        half = dim // 2
        k = torch.arange(half, dtype=torch.float32, device=t.device)
        freqs = torch.exp(-math.log(max_period) * k / half)
        args = t.float()[:, None] * freqs[None]
        emb = torch.cat([args.cos(), args.sin()], dim=-1)
        if dim % 2:
            emb = F.pad(emb, (0, 1))
        return emb

    def forward(self, t: torch.Tensor) -> torch.Tensor:
        return self.mlp(self.timestep_embedding(t, self.frequency_embedding_size))


class LabelEmbedder(nn.Module):
    """num_classes + 1 embeddings (the last one is the null label used for guidance) (local_thc.py:203-210)."""

    def __init__(self, num_classes: int, hidden_size: int) -> None:
        super().__init__()
        self.num_classes = num_classes
        self.embedding_table = nn.Embedding(num_classes + 1, hidden_size)

    def forward(self, labels: torch.Tensor) -> torch.Tensor:
        return self.embedding_table(labels)


class WorkspaceAttention(nn.Module):
    """QK-RMSNorm multi-head self-attention with 2-D RoPE over the workspace tokens (local_thc.py:213-256)."""

    def __init__(
        self,
        dim: int,
        num_heads: int = 12,
        qkv_bias: bool = True,
        qk_norm: bool = True,
        attn_drop: float = 0.0,
        proj_drop: float = 0.0,
        attn_backend: str = "flash",
    ) -> None:
        super().__init__()
        if dim % num_heads != 0:
            raise ValueError(f"dim={dim} must be divisible by num_heads={num_heads}")
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.qkv = CastLinear(dim, dim * 3, bias=qkv_bias)
        self.q_norm = RMSNorm(self.head_dim) if qk_norm else nn.Identity()
        self.k_norm = RMSNorm(self.head_dim) if qk_norm else nn.Identity()
        self.attn_drop = nn.Dropout(attn_drop)
        self.proj = CastLinear(dim, dim)
        self.proj_drop = nn.Dropout(proj_drop)
        self.attn_backend = attn_backend
        # q/k norm + RoPE + attention as one HIP pass (jit_thc::qk_norm_rope_attention) where it applies
        self.fused_attention = True

    def _backends(self):
        table = {
            "flash": [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION, SDPBackend.MATH],
            "efficient": [SDPBackend.EFFICIENT_ATTENTION, SDPBackend.MATH],
            "math": [SDPBackend.MATH],
        }
        return sdpa_kernel(table[self.attn_backend]) if self.attn_backend in table else nullcontext()

    def _fused_qk(self, qkv: torch.Tensor, rope: VisionRotaryEmbeddingFast) -> bool:
        """Whether jit_thc::qk_norm_rope covers this call (GPU, head_dim 64, RMSNorm q/k norms, a full RoPE table)."""
        return (
            qkv.is_cuda
            and qkv.dtype in (torch.bfloat16, torch.float16, torch.float32)
            and self.head_dim == ops_branch.QK_HEAD_DIM
            and isinstance(self.q_norm, RMSNorm)
            and isinstance(self.k_norm, RMSNorm)
            and self.q_norm.eps == self.k_norm.eps
            and tuple(rope.freqs_cos.shape) == (qkv.shape[1], self.head_dim)
        )

    def _fused_attn(self, qkv5: torch.Tensor) -> bool:
        """Whether jit_thc::qk_norm_rope_attention replaces the SDPA call: switched on, a fast SDPA backend
        requested (not the math reference path), no attention dropout active, a supported shape and dtype."""
        return (
            self.fused_attention
            and self.attn_backend in ("flash", "efficient")
            and not (self.training and self.attn_drop.p > 0.0)
            and ops_branch.attention_supported(qkv5)
        )

    def forward(self, x: torch.Tensor, rope: VisionRotaryEmbeddingFast) -> torch.Tensor:
        b, n, c = x.shape
        qkv = self.qkv(x)
        if self._fused_qk(qkv, rope):
            qkv5 = qkv.view(b, n, 3, self.num_heads, self.head_dim)
            if self._fused_attn(qkv5):
                # q/k norm + rope and the attention itself in one matrix-core pass, o as [B, N, H, D]
                cos, sin = rope.tables(qkv.dtype)  # the values the kernel rounds the tables to, cast once
                o = ops_branch.qk_norm_rope_attention(
                    qkv5, self.q_norm.weight, self.k_norm.weight, cos, sin, self.q_norm.eps
                )
                return self.proj_drop(self.proj(o.reshape(b, n, c)))
            # one HIP pass for q_norm + rope and k_norm + rope, with the eager sequence's roundings
            q, k = ops_branch.qk_norm_rope(
                qkv5, self.q_norm.weight, self.k_norm.weight, rope.freqs_cos, rope.freqs_sin, self.q_norm.eps
            )
            q, k, v = q.transpose(1, 2), k.transpose(1, 2), qkv5[:, :, 2].transpose(1, 2)
        else:
            q, k, v = qkv.view(b, n, 3, self.num_heads, self.head_dim).permute(2, 0, 3, 1, 4).unbind(0)
            q = rope(self.q_norm(q))
            k = rope(self.k_norm(k))
        with self._backends():
            o = F.scaled_dot_product_attention(q, k, v, dropout_p=self.attn_drop.p if self.training else 0.0)
        return self.proj_drop(self.proj(o.transpose(1, 2).reshape(b, n, c)))


class SwiGLUFFN(nn.Module):
    """SwiGLU MLP with hidden width int(hidden_dim * 2 / 3); w12 output split (gate, value) (local_thc.py:259-269)."""

    def __init__(self, dim: int, hidden_dim: int, drop: float = 0.0, bias: bool = True) -> None:
        super().__init__()
        hidden = int(hidden_dim * 2 / 3)
        self.w12 = CastLinear(dim, 2 * hidden, bias=bias)
        self.w3 = CastLinear(hidden, dim, bias=bias)
        self.ffn_dropout = nn.Dropout(drop)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = self.w12(x)
        if h.is_cuda and h.dtype in (torch.bfloat16, torch.float16, torch.float32) and h.shape[-1] % 16 == 0:
            act = ops_branch.swiglu(h)  # silu(gate) * value in one HIP pass, eager roundings
        else:
            gate, value = h.chunk(2, dim=-1)
            act = F.silu(gate) * value
        return self.w3(self.ffn_dropout(act))


class WorkspaceSharedAdaLNBranch(nn.Module):
    """Attention + SwiGLU branch on the workspace, modulated by the shared [B, 6C] AdaLN vector (local_thc.py:302-323).

    Returns the branch update dZ = gate_msa * attn(...) + gate_mlp * mlp(...).
    """

    def __init__(
        self,
        hidden_size: int,
        num_heads: int,
        mlp_ratio: float = 4.0,
        attn_drop: float = 0.0,
        proj_drop: float = 0.0,
        attn_backend: str = "flash",
    ) -> None:
        super().__init__()
        self.norm1 = RMSNorm(hidden_size, eps=1e-6)
        self.attn = WorkspaceAttention(hidden_size, num_heads, attn_drop=attn_drop, proj_drop=proj_drop, attn_backend=attn_backend)
        self.norm2 = RMSNorm(hidden_size, eps=1e-6)
        self.mlp = SwiGLUFFN(hidden_size, int(hidden_size * mlp_ratio), drop=proj_drop)

    def forward(self, z: torch.Tensor, t6: torch.Tensor, rope: VisionRotaryEmbeddingFast) -> torch.Tensor:
        sh_a, sc_a, g_a, sh_m, sc_m, g_m = t6.chunk(6, dim=-1)
        a = self.attn(norm_modulate(self.norm1, z, sh_a, sc_a), rope)
        if self.fused_gates(z, a, t6):
            # d_attn = g_a * a, z + d_attn and its pre-norm in one HIP pass; d_attn + g_m * mlp in another
            d_attn, h = ops_branch.gate_add_norm_modulate(z, a, g_a, self.norm2.weight, sh_m, sc_m, self.norm2.eps)
            return ops_branch.gate_residual(d_attn, g_m, self.mlp(h))
        d_attn = g_a.unsqueeze(1) * a
        d_mlp = g_m.unsqueeze(1) * self.mlp(norm_modulate(self.norm2, z + d_attn, sh_m, sc_m))
        return d_attn + d_mlp

    @staticmethod
    def fused_gates(z: torch.Tensor, a: torch.Tensor, t6: torch.Tensor) -> bool:
        """The gated residuals run as HIP passes: GPU, [B, N, C] with C % 8 == 0 and C <= 2048, one dtype."""
        return z.is_cuda and z.dim() == 3 and a.dtype == z.dtype == t6.dtype and z.shape[-1] % 8 == 0 and z.shape[-1] <= 2048

    def parts(
        self, z: torch.Tensor, t6: torch.Tensor, rope: VisionRotaryEmbeddingFast, y1: torch.Tensor | None = None
    ) -> tuple[torch.Tensor, torch.Tensor] | None:
        """(g_a * attn, mlp output): forward() without its last gated residual, or None where the gated residuals
        are not HIP passes.  y1: this branch's first pre-norm output when the caller has computed it."""
        sh_a, sc_a, g_a, sh_m, sc_m, _ = t6.chunk(6, dim=-1)
        a = self.attn(y1 if y1 is not None else norm_modulate(self.norm1, z, sh_a, sc_a), rope)
        if not self.fused_gates(z, a, t6):
            return None
        d_attn, h = ops_branch.gate_add_norm_modulate(z, a, g_a, self.norm2.weight, sh_m, sc_m, self.norm2.eps)
        return d_attn, self.mlp(h)


class FinalLayerSharedAdaLN(nn.Module):
    """RMSNorm, shared [B, 2C] modulation (shift, scale), linear to patch pixels (local_thc.py:865-873)."""

    def __init__(self, hidden_size: int, patch_size: int, out_channels: int) -> None:
        super().__init__()
        self.norm_final = RMSNorm(hidden_size)
        self.linear = CastLinear(hidden_size, patch_size * patch_size * out_channels, bias=True)

    def forward(self, x: torch.Tensor, t2: torch.Tensor) -> torch.Tensor:
        shift, scale = t2.chunk(2, dim=1)
        return self.linear(norm_modulate(self.norm_final, x, shift, scale))


class WorkspaceJiTBranch(WorkspaceSharedAdaLNBranch):
    """The workspace branch with its own AdaLN head (local_thc.py:270-297): t6 = adaLN_modulation(c), then the
    shared-AdaLN branch's attention + SwiGLU update."""

    def __init__(
        self,
        hidden_size: int,
        num_heads: int,
        mlp_ratio: float = 4.0,
        attn_drop: float = 0.0,
        proj_drop: float = 0.0,
        attn_backend: str = "flash",
    ) -> None:
        super().__init__(hidden_size, num_heads, mlp_ratio, attn_drop, proj_drop, attn_backend)
        self.adaLN_modulation = nn.Sequential(nn.SiLU(), CastLinear(hidden_size, 6 * hidden_size, bias=True))

    def forward(self, z: torch.Tensor, c: torch.Tensor, rope: VisionRotaryEmbeddingFast) -> torch.Tensor:
        return self.forward_with_modulation(z, self.adaLN_modulation(c), rope)

    def forward_with_modulation(self, z: torch.Tensor, t6: torch.Tensor, rope: VisionRotaryEmbeddingFast) -> torch.Tensor:
        return super().forward(z, t6, rope)


class FinalLayer(FinalLayerSharedAdaLN):
    """The decoder with its own AdaLN head (local_thc.py:853-862): (shift, scale) = adaLN_modulation(c)."""

    def __init__(self, hidden_size: int, patch_size: int, out_channels: int) -> None:
        super().__init__(hidden_size, patch_size, out_channels)
        self.adaLN_modulation = nn.Sequential(nn.SiLU(), CastLinear(hidden_size, 2 * hidden_size, bias=True))

    def forward(self, x: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
        return super().forward(x, self.adaLN_modulation(c))


class SharedReadLocalTHCSharedAdaLNJiTBlock(nn.Module):
    """One layer: the layer's local write and its workspace branch (local_thc.py:1286-1328)."""

    def __init__(
        self,
        hidden_size: int,
        num_heads: int,
        high_grid: int,
        workspace_grid: int = 16,
        pool_groups: int | None = None,
        mlp_ratio: float = 4.0,
        attn_drop: float = 0.0,
        proj_drop: float = 0.0,
        attn_backend: str = "flash",
    ) -> None:
        super().__init__()
        pool_groups = hidden_size if pool_groups is None else pool_groups
        self.write = LayerLocalWrite(high_grid, workspace_grid, hidden_size, pool_groups)
        self.branch = WorkspaceSharedAdaLNBranch(hidden_size, num_heads, mlp_ratio, attn_drop, proj_drop, attn_backend)

    @property
    def read(self) -> LayerLocalWrite:
        """Old checkpoint name of the layer's write module."""
        return self.write

    def forward_naive(self, x_hi, t6, rope, shared_read: SharedLocalRead) -> torch.Tensor:
        z = shared_read.read(x_hi)
        return self.write.write_add(x_hi, self.branch(z, t6, rope))

    def branch_update(self, z: torch.Tensor, t6: torch.Tensor, rope: VisionRotaryEmbeddingFast) -> torch.Tensor:
        return self.branch(z, t6, rope)

    def lazy_workspace_update(self, z: torch.Tensor, dz: torch.Tensor, shared_read: SharedLocalRead) -> torch.Tensor:
        """Z_{l+1} = Z_l + gamma_l * dZ_l; gamma_l from the shared read and this layer's write weights."""
        gamma = self.write.gamma_from_alpha(shared_read.alpha(dtype=dz.dtype))
        return ops.lazy_workspace_update(z, dz, gamma)

    def lazy_workspace_step(
        self,
        z: torch.Tensor,
        dz: torch.Tensor,
        shared_read: SharedLocalRead,
        gamma: torch.Tensor | None = None,
        split: bool = False,
    ) -> tuple[torch.Tensor, ...]:
        """(lazy_workspace_update(z, dz), dz) for the lazy forward, where dz is also materialised at the end;
        the backward writes dz's whole gradient in one recurrence-backward pass (ops.lazy_workspace_step).
        gamma: this layer's gamma_from_alpha(shared_read.alpha(dz.dtype)) when the caller has computed it.
        split: return (z_next, z_next for the next block's branch, dz), whose backward also sums z_next's
        two gradients in that pass."""
        if overridden(self, "lazy_workspace_update", SharedReadLocalTHCSharedAdaLNJiTBlock):
            # a replaced reference hook (local_thc.py:1325) defines the step; gamma is its business
            z_next = self.lazy_workspace_update(z, dz, shared_read)
            return (z_next, z_next, dz) if split else (z_next, dz)
        if gamma is None:
            gamma = self.write.gamma_from_alpha(shared_read.alpha(dtype=dz.dtype))
        return ops.lazy_workspace_step(z, dz, gamma, split)


def migrate_lthc_state_dict_keys(state_dict: dict) -> dict:
    """Old checkpoint key names -> current ones (local_thc.py:41-61): the old code called the read 'write'."""
    rules = (
        (r"shared_write\.", "shared_read."),
        (r"blocks\.(\d+)\.read\.", r"blocks.\1.write."),
        (r"\.write_logits", ".read_logits"),
        (r"\.read_weight", ".write_weight"),
    )
    out = {}
    for key, value in state_dict.items():
        for pat, rep in rules:
            key = re.sub(pat, rep, key)
        out[key] = value
    return out


class BatchedWeightCast:
    """Mixin for the models of this package: their inference forwards under autocast convert every linear and
    patch-embedding weight in one launch instead of one conversion per layer."""

    batched_weight_cast = True

    def _conversion_targets(self) -> list[tuple[nn.Module, list[torch.Tensor]]]:
        """Modules whose weights autocast would convert on every forward, with the tensors it would convert."""
        out: list[tuple[nn.Module, list[torch.Tensor]]] = [
            (m, [m.weight, m.bias] if m.bias is not None else [m.weight])
            for m in self.modules()
            if isinstance(m, CastLinear)
        ]
        pe = self.x_embedder
        embed = pe.cast_targets() if hasattr(pe, "cast_targets") else None
        if embed is not None:
            out.append((pe, embed))
        return out

    @contextmanager
    def _converted_weights(self):
        """Under a bf16 / fp16 CUDA autocast without autograd and with fp32 parameters (inference), convert every
        linear weight once, in one launch (ops.BatchedCast), for this forward: the values autocast's ~150
        per-layer conversions would produce.  Otherwise (training, no autocast, 16-bit parameters) a no-op."""
        targets = self._conversion_targets() if self.batched_weight_cast else []
        dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else None
        tensors = [t for _, ts in targets for t in ts]
        usable = (
            bool(tensors)
            and dt in (torch.bfloat16, torch.float16)
            and not torch.is_grad_enabled()
            and all(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous() for t in tensors)
        )
        bc = self.__dict__.get("_batched_cast") if usable else None
        key = (dt, tuple((t.data_ptr(), t.numel()) for t in tensors)) if usable else None
        if usable and (bc is None or bc.key != key):
            if torch.cuda.is_current_stream_capturing():  # the table is built eagerly, outside a capture
                usable = False
            else:
                bc = ops.BatchedCast(tensors, dt)
                self.__dict__["_batched_cast"] = bc
        if not usable:
            yield
            return
        outs = bc()
        i = 0
        for m, ts in targets:
            m.__dict__["_cast"] = tuple(outs[i : i + len(ts)])
            i += len(ts)
        try:
            yield
        finally:
            for m, _ in targets:
                m.__dict__.pop("_cast", None)


def _standard_decoder(fl: nn.Module) -> bool:
    """fl is this package's shared-AdaLN or per-block-AdaLN decoder with nothing replaced."""
    return (
        type(fl) in (FinalLayerSharedAdaLN, FinalLayer)
        and "forward" not in fl.__dict__
        and type(fl.norm_final) is RMSNorm
        and fl.linear.bias is not None
    )


def decoder_records_grad(fl: nn.Module, x: torch.Tensor, cond: torch.Tensor) -> bool:
    """Autograd would record decoder fl on x: then the eager decoder runs, since jit_thc::decoder_head's backward
    replays the eager sequence and a training step with it took 5.5 ms longer (LTHC-B/4, B=64: 61.9 against
    56.3 ms)."""
    return torch.is_grad_enabled() and (
        x.requires_grad or cond.requires_grad or any(p.requires_grad for p in fl.parameters())
    )


def _decoder_modulation(fl: nn.Module, cond: torch.Tensor) -> torch.Tensor:
    """The [B, 2C] (shift, scale) a standard decoder applies for cond (local_thc.py:853-873)."""
    return cond if type(fl) is FinalLayerSharedAdaLN else fl.adaLN_modulation(cond)


def decode_output(model: nn.Module, x_hi: torch.Tensor, cond: torch.Tensor) -> torch.Tensor:
    """unpatchify(final_layer(X, cond)) for X [B, H, H, C].  With a standard decoder, 16-bit X on the GPU, 4x4
    patches and no autograd recording: RMSNorm, modulation, linear layer and unpatchify in one jit_thc::decoder_head
    pass."""
    fl = model.final_layer
    b, hh, wh, c = x_hi.shape
    x = x_hi.reshape(b, hh * wh, c)
    fusable = getattr(model, "fused_decoder", True) and _standard_decoder(fl) and model.patch_size == 4
    if fusable and not decoder_records_grad(fl, x, cond):
        if ops.decoder_head_supported(x, fl.linear.weight):
            t2 = _decoder_modulation(fl, cond)
            if t2.dtype == x.dtype:
                shift, scale = t2.chunk(2, dim=1)
                lw, lb = fl.linear.__dict__.get("_cast") or (fl.linear.weight, fl.linear.bias)
                return ops.decoder_head(x, fl.norm_final.weight, shift, scale, lw, lb, fl.norm_final.eps, hh, 4)
            return model.unpatchify(FinalLayerSharedAdaLN.forward(fl, x, t2))
    return model.unpatchify(fl(x, cond))


def materialise_decode_output(
    model: nn.Module, x0: torch.Tensor, dz_list: list[torch.Tensor], betas: list[torch.Tensor], cond: torch.Tensor
) -> torch.Tensor | None:
    """decode_output(model, x0 + sum_l P_{betas[l]}(dz_list[l]), cond) as one jit_thc::final_accumulate_decoder_head
    pass, X_L never written, where that applies: no autograd, a standard decoder, 16-bit operands of one dtype on the
    GPU and the pass's shapes.  None elsewhere: the caller materialises and decodes."""
    fl = model.final_layer
    if not (
        getattr(model, "fused_materialise_decoder", True)
        and getattr(model, "fused_decoder", True)
        and not torch.is_grad_enabled()
        and _standard_decoder(fl)
        and all(dz.dtype == x0.dtype and dz.is_cuda for dz in dz_list)
        and ops.materialise_decoder_supported(x0, dz_list, fl.linear.weight, model.patch_size)
    ):
        return None
    t2 = _decoder_modulation(fl, cond)
    if t2.dtype != x0.dtype:
        return None
    shift, scale = t2.chunk(2, dim=1)
    lw, lb = fl.linear.__dict__.get("_cast") or (fl.linear.weight, fl.linear.bias)
    return ops.final_accumulate_decoder_head(
        x0, list(dz_list), list(betas), fl.norm_final.weight, shift, scale, lw, lb, fl.norm_final.eps, model.patch_size
    )


class SharedReadLocalTHCSharedAdaLNJiT(BatchedWeightCast, nn.Module):
    """LTHC JiT with a depth-shared read, per-layer writes and shared AdaLN (local_thc.py:883-1007, :1331-1394).

    forward_lazy: read X0 once, run the blocks on the workspace with the exact
    recurrence Z_{l+1} = Z_l + gamma_l dZ_l, materialise X_L once, decode.
    forward_naive: per block read X_l, branch, write back X_{l+1} = X_l + P_l dZ_l.
    """

    block_cls = SharedReadLocalTHCSharedAdaLNJiTBlock

    def __init__(
        self,
        input_size: int = 256,
        patch_size: int = 4,
        in_channels: int = 3,
        hidden_size: int = 768,
        depth: int = 12,
        num_heads: int = 12,
        mlp_ratio: float = 4.0,
        attn_drop: float = 0.0,
        proj_drop: float = 0.0,
        num_classes: int = 1000,
        bottleneck_dim: int = 128,
        workspace_grid: int = 16,
        pool_groups: int | None = None,
        attn_backend: str = "flash",
        use_lazy: bool = True,
    ) -> None:
        super().__init__()
        high_grid = input_size // patch_size
        if high_grid % workspace_grid != 0:
            raise ValueError(f"input_size/patch_size={high_grid} must be divisible by workspace_grid={workspace_grid}")
        self.input_size = input_size
        self.patch_size = patch_size
        self.in_channels = in_channels
        self.out_channels = in_channels
        self.hidden_size = hidden_size
        self.depth = depth
        self.num_heads = num_heads
        self.num_classes = num_classes
        self.workspace_grid = workspace_grid
        self.high_grid = high_grid
        self.num_high_tokens = high_grid * high_grid
        self.num_workspace_tokens = workspace_grid * workspace_grid
        self.pool_groups = hidden_size if pool_groups is None else pool_groups

        self.t_embedder = TimestepEmbedder(hidden_size)
        self.y_embedder = LabelEmbedder(num_classes, hidden_size)
        self.x_embedder = BottleneckPatchEmbedNHWC(input_size, patch_size, in_channels, bottleneck_dim, hidden_size)
        self.workspace_rope = VisionRotaryEmbeddingFast(hidden_size // num_heads // 2, workspace_grid)
        quarter = depth // 4
        self.blocks = nn.ModuleList(
            self.block_cls(
                hidden_size=hidden_size,
                num_heads=num_heads,
                high_grid=high_grid,
                workspace_grid=workspace_grid,
                pool_groups=self.pool_groups,
                mlp_ratio=mlp_ratio,
                attn_drop=attn_drop if quarter <= i < 3 * quarter else 0.0,
                proj_drop=proj_drop if quarter <= i < 3 * quarter else 0.0,
                attn_backend=attn_backend,
            )
            for i in range(depth)
        )
        self.final_layer = FinalLayerSharedAdaLN(hidden_size, patch_size, self.out_channels)
        self.shared_adaLN_modulation = nn.Sequential(nn.SiLU(), CastLinear(hidden_size, 6 * hidden_size, bias=True))
        self.shared_final_modulation = nn.Sequential(nn.SiLU(), CastLinear(hidden_size, 2 * hidden_size, bias=True))
        self.initialize_weights()
        self.shared_read = SharedLocalRead(high_grid, workspace_grid, hidden_size, self.pool_groups, use_softmax_write=True)
        self.use_lazy = bool(use_lazy)
        # decoder head as one HIP pass (jit_thc::decoder_head) where it applies
        self.fused_decoder = True
        # inference under autocast with fp32 parameters: all weight conversions in one launch
        self.batched_weight_cast = True
        # inference: each block's last gated residual, its recurrence step and the next block's first pre-norm in
        # one HIP pass (jit_thc::block_tail)
        self.fused_block_tail = True
        # inference: the final materialisation with the decoder's norm, modulation and linear layer in its
        # epilogue, X_L never written (jit_thc::final_accumulate_decoder_head)
        self.fused_materialise_decoder = True

    # -- initialisation (local_thc.py:944-970, :1004-1007) ------------------------------------------
    def initialize_weights(self) -> None:
        for m in self.modules():
            if isinstance(m, nn.Linear):
                nn.init.xavier_uniform_(m.weight)
                if m.bias is not None:
                    nn.init.zeros_(m.bias)
        for conv in (self.x_embedder.proj1, self.x_embedder.proj2):
            nn.init.xavier_uniform_(conv.weight.data.view(conv.weight.shape[0], -1))
        nn.init.zeros_(self.x_embedder.proj2.bias)
        nn.init.normal_(self.y_embedder.embedding_table.weight, std=0.02)
        nn.init.normal_(self.t_embedder.mlp[0].weight, std=0.02)
        nn.init.normal_(self.t_embedder.mlp[2].weight, std=0.02)
        nn.init.zeros_(self.final_layer.linear.weight)
        nn.init.zeros_(self.final_layer.linear.bias)
        for head in (self.shared_adaLN_modulation[-1], self.shared_final_modulation[-1]):
            nn.init.zeros_(head.weight)
            nn.init.zeros_(head.bias)

    def load_state_dict(self, state_dict, strict: bool = True, assign: bool = False):
        return super().load_state_dict(migrate_lthc_state_dict_keys(state_dict), strict=strict, assign=assign)

    @property
    def shared_write(self) -> SharedLocalRead:
        """Old name of the shared read."""
        return self.shared_read

    def unpatchify(self, x: torch.Tensor) -> torch.Tensor:
        """[B, h*w, p*p*c] -> [B, c, h*p, w*p] (local_thc.py:972-980)."""
        c, p = self.out_channels, self.patch_size
        h = w = math.isqrt(x.shape[1])
        if h * w != x.shape[1]:
            raise ValueError(f"token count {x.shape[1]} is not square")
        x = x.reshape(x.shape[0], h, w, p, p, c).permute(0, 5, 1, 3, 2, 4)
        return x.reshape(x.shape[0], c, h * p, w * p)

    # -- interface ---------------------------------------------------------------------------------
    def final_accumulate_reference(self, x0: torch.Tensor, dz_list: list[torch.Tensor]) -> torch.Tensor:
        """X_L = X0 + sum_l P_l(dZ_l) in one pass (the reference's generic loop, local_thc.py:1368-1372), the
        layers passed as lists so no dZ stack is built."""
        if len(dz_list) != len(self.blocks):
            raise ValueError(f"expected {len(self.blocks)} updates, got {len(dz_list)}")
        betas = [blk.write.channel_beta(dtype=torch.float32) for blk in self.blocks]
        return ops.final_accumulate_list(x0, list(dz_list), betas)

    def _conditioning(self, t: torch.Tensor, y: torch.Tensor):
        c = self.t_embedder(t) + self.y_embedder(y)
        return self.shared_adaLN_modulation(c), self.shared_final_modulation(c)

    def _decode(self, x_hi: torch.Tensor, t2: torch.Tensor) -> torch.Tensor:
        b, hh, wh, c_dim = x_hi.shape
        x = x_hi.reshape(b, hh * wh, c_dim)
        fl = self.final_layer
        if (
            self.fused_decoder
            and t2.dtype == x.dtype
            and isinstance(fl.norm_final, RMSNorm)
            and fl.linear.bias is not None
            and self.patch_size == 4
            and not decoder_records_grad(fl, x, t2)
            and ops.decoder_head_supported(x, fl.linear.weight)
        ):
            # RMSNorm + modulate + linear + unpatchify in one pass (jit_thc::decoder_head): y never reaches memory
            shift, scale = t2.chunk(2, dim=1)
            lw, lb = fl.linear.__dict__.get("_cast") or (fl.linear.weight, fl.linear.bias)
            return ops.decoder_head(x, fl.norm_final.weight, shift, scale, lw, lb, fl.norm_final.eps, hh, self.patch_size)
        return self.unpatchify(fl(x, t2))

    def _materialise_decode(self, x0: torch.Tensor, dz_list: list[torch.Tensor], t2: torch.Tensor) -> torch.Tensor:
        """decode(X_L) for X_L = x0 + sum_l P_l(dZ_l).  Under no-grad on the GPU, with the standard final layer and
        materialisation hooks, one pass forms X_L per token and feeds it to the decoder's norm, modulation and linear
        layer without writing it (jit_thc::final_accumulate_decoder_head); otherwise X_L, then the decoder."""
        fl = self.final_layer
        if (
            self.fused_materialise_decoder
            and self.fused_decoder
            and not torch.is_grad_enabled()
            and type(fl) is FinalLayerSharedAdaLN
            and "forward" not in fl.__dict__
            and isinstance(fl.norm_final, RMSNorm)
            and fl.linear.bias is not None
            and "final_accumulate_reference" not in self.__dict__
            and (
                type(self).final_accumulate_reference is SharedReadLocalTHCSharedAdaLNJiT.final_accumulate_reference
                # the fused-final-12 hook takes exactly 12 layers: other depths reach its ValueError below
                or (
                    type(self).final_accumulate_reference
                    is SharedReadFusedFinal12LocalTHCSharedAdaLNJiT.final_accumulate_reference
                    and len(dz_list) == 12
                )
            )
            and len(dz_list) == len(self.blocks)
            and t2.dtype == x0.dtype
            and all(dz.dtype == x0.dtype and dz.is_cuda for dz in dz_list)
            and ops.materialise_decoder_supported(x0, dz_list, fl.linear.weight, self.patch_size)
        ):
            betas = [blk.write.channel_beta(dtype=torch.float32) for blk in self.blocks]
            shift, scale = t2.chunk(2, dim=1)
            lw, lb = fl.linear.__dict__.get("_cast") or (fl.linear.weight, fl.linear.bias)
            return ops.final_accumulate_decoder_head(
                x0, list(dz_list), betas, fl.norm_final.weight, shift, scale, lw, lb, fl.norm_final.eps, self.patch_size
            )
        return self._decode(self.final_accumulate_reference(x0, dz_list), t2)

    def forward_lazy(self, x: torch.Tensor, t: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        t6, t2 = self._conditioning(t, y)
        # local_thc.py:1376-1385 (read once, one branch + recurrence per block, one materialisation).  The read
        # and the recurrence steps are the fused-backward forms: same values, x0's, each dZ_l's and each Z_l's
        # gradient from one kernel instead of a kernel plus autograd's add.
        x0, z = self.shared_read.read_with_residual(self.x_embedder(x))
        if self._tail_fusable(z):
            dz_list = self._blocks_fused_tail(z, t6)
            if dz_list is not None:
                return self._materialise_decode(x0, dz_list, t2)
        zb = z  # the next branch's input: z itself, or the step's branch output (same values)
        dz_list, gammas = [], None
        for i, block in enumerate(self.blocks):
            dz = block.branch_update(zb, t6, self.workspace_rope)
            if i == 0:
                gammas = self._all_gammas(dz)
            if gammas is None:  # the reference's hook signature
                z, dz = block.lazy_workspace_step(z, dz, self.shared_read)
                zb = z
            else:
                z, zb, dz = block.lazy_workspace_step(z, dz, self.shared_read, gammas[i], split=True)
            dz_list.append(dz)
        return self._materialise_decode(x0, dz_list, t2)

    def _tail_fusable(self, z: torch.Tensor) -> bool:
        """Inference on the GPU with the standard blocks, hooks, branch and ungrouped weights: jit_thc::block_tail
        applies."""
        std = SharedReadLocalTHCSharedAdaLNJiTBlock
        if not (
            self.fused_block_tail
            and not torch.is_grad_enabled()
            and z.is_cuda
            and len(self.blocks) > 1
            and self.shared_read.group_dim == 1
        ):
            return False
        for blk in self.blocks:  # a plain loop (torch.compile traces it without a graph break)
            if not (
                blk.write.group_dim == 1
                and type(blk) is std
                and "branch_update" not in blk.__dict__
                and "lazy_workspace_step" not in blk.__dict__
                and "lazy_workspace_update" not in blk.__dict__
                and type(blk.branch) is WorkspaceSharedAdaLNBranch
                and "forward" not in blk.branch.__dict__
            ):
                return False
        return True

    def _blocks_fused_tail(self, z: torch.Tensor, t6: torch.Tensor) -> list[torch.Tensor] | None:
        """The block loop of forward_lazy with each block's gate_residual, its recurrence step and the next block's
        first pre-norm as one jit_thc::block_tail pass: the same values as the hook path.  Returns the dZ list, or
        None (nothing computed that the caller keeps) when the first block's gated residuals are not HIP passes."""
        sh_a, sc_a, _, _, _, g_m = t6.chunk(6, dim=-1)
        dz_list, gammas, y1 = [], None, None
        nb = len(self.blocks)
        for i, block in enumerate(self.blocks):
            parts = block.branch.parts(z, t6, self.workspace_rope, y1)
            if parts is None:
                if i == 0:
                    return None
                raise RuntimeError("the blocks' gated residuals changed path between blocks")
            d_attn, mo = parts
            if i == 0:
                gammas = self._all_gammas(d_attn)
                if gammas is None:
                    return None
            if i + 1 < nb:
                n1 = self.blocks[i + 1].branch.norm1
                dz, z, y1 = ops_branch.block_tail(z, d_attn, g_m, mo, gammas[i], n1.weight, sh_a, sc_a, n1.eps)
            else:  # the last step's Z_L feeds nothing
                dz = ops_branch.gate_residual(d_attn, g_m, mo)
            dz_list.append(dz)
        return dz_list

    def _all_gammas(self, dz: torch.Tensor) -> list[torch.Tensor] | None:
        """Every block's gamma_from_alpha(shared_read.alpha(dz.dtype)) in one launch (ops.lazy_gamma_rounded: the
        same dtype sequence), or None where it does not apply (CPU, grouped write weights, another block type)."""
        writes = [blk.write for blk in self.blocks]
        std = SharedReadLocalTHCSharedAdaLNJiTBlock
        if not dz.is_cuda or overridden(self.shared_read, "alpha", SharedLocalRead) or self.shared_read.group_dim != 1:
            return None
        for blk in self.blocks:  # a plain loop (torch.compile traces it without a graph break)
            # no block replaces a hook the gammas come from (subclass or instance override)
            if (
                overridden(blk, "lazy_workspace_step", std)
                or overridden(blk, "lazy_workspace_update", std)
                or overridden(blk.write, "gamma_from_alpha", LayerLocalWrite)
                or overridden(blk.write, "beta", LayerLocalWrite)
                or blk.write.group_dim != 1
            ):
                return None
        return list(ops.lazy_gamma_rounded(self.shared_read.alpha(), [w.write_weight for w in writes], dz.dtype).unbind(0))

    def forward_naive(self, x: torch.Tensor, t: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        t6, t2 = self._conditioning(t, y)
        x_hi = self.x_embedder(x)
        for block in self.blocks:
            x_hi = block.forward_naive(x_hi, t6, self.workspace_rope, self.shared_read)
        return self._decode(x_hi, t2)

    def forward(self, x: torch.Tensor, t: torch.Tensor, y: torch.Tensor, use_lazy: bool | None = None) -> torch.Tensor:
        lazy = self.use_lazy if use_lazy is None else use_lazy
        if torch.compiler.is_compiling():
            # under torch.compile the compiler fuses autocast's weight conversions itself; the one-launch table
            # (built eagerly, kept on the module) is for eager and HIP-graph forwards
            return self.forward_lazy(x, t, y) if lazy else self.forward_naive(x, t, y)
        with self._converted_weights():
            return self.forward_lazy(x, t, y) if lazy else self.forward_naive(x, t, y)


class SharedReadFusedFinalLocalTHCSharedAdaLNJiT(SharedReadLocalTHCSharedAdaLNJiT):
    """Any-depth form whose materialisation is the stacked op over [L,B,M,C] dZ and [L,C,16] write weights
    (local_thc.py:1397-1410)."""

    def final_accumulate_reference(self, x0: torch.Tensor, dz_list: list[torch.Tensor]) -> torch.Tensor:
        dz_stack = torch.stack(dz_list, dim=0).contiguous()
        beta_stack = torch.stack([blk.write.write_weight for blk in self.blocks], dim=0).contiguous()
        return ops.final_accumulate_b4_traceable(x0, dz_stack, beta_stack)


class SharedReadFusedFinal12LocalTHCSharedAdaLNJiT(SharedReadLocalTHCSharedAdaLNJiT):
    """Depth-12 form whose materialisation is the 12-pointer op (local_thc.py:1413-1420)."""

    def final_accumulate_reference(self, x0: torch.Tensor, dz_list: list[torch.Tensor]) -> torch.Tensor:
        if len(dz_list) != 12 or len(self.blocks) != 12:
            raise ValueError("SharedReadFusedFinal12LocalTHCSharedAdaLNJiT requires depth=12")
        betas = [blk.write.channel_beta() for blk in self.blocks]
        return ops.final_accumulate_b4_12_traceable(x0, *dz_list, *betas)


# Old class names (local_thc.py:1428-1431).
SharedWriteLocalTHCSharedAdaLNJiTBlock = SharedReadLocalTHCSharedAdaLNJiTBlock
SharedWriteLocalTHCSharedAdaLNJiT = SharedReadLocalTHCSharedAdaLNJiT
SharedWriteFusedFinalLocalTHCSharedAdaLNJiT = SharedReadFusedFinalLocalTHCSharedAdaLNJiT
SharedWriteFusedFinal12LocalTHCSharedAdaLNJiT = SharedReadFusedFinal12LocalTHCSharedAdaLNJiT


def SharedRead_FusedFinal12_LocalTHC_SharedAdaLN_JiT_B_4(**kwargs) -> SharedReadFusedFinal12LocalTHCSharedAdaLNJiT:
    """LTHC-B/4: patch 4, hidden 768, depth 12, 12 heads, bottleneck 128, 16x16 workspace (local_thc.py:1705-1719)."""
    kwargs.setdefault("pool_groups", 768)
    return SharedReadFusedFinal12LocalTHCSharedAdaLNJiT(
        patch_size=4, hidden_size=768, depth=12, num_heads=12, bottleneck_dim=128, workspace_grid=16, **kwargs
    )


def SharedRead_FusedFinal_LocalTHC_SharedAdaLN_JiT_B_4(**kwargs) -> SharedReadFusedFinalLocalTHCSharedAdaLNJiT:
    kwargs.setdefault("pool_groups", 768)
    return SharedReadFusedFinalLocalTHCSharedAdaLNJiT(
        patch_size=4, hidden_size=768, depth=12, num_heads=12, bottleneck_dim=128, workspace_grid=16, **kwargs
    )


def SharedRead_LocalTHC_SharedAdaLN_JiT_B_4(**kwargs) -> SharedReadLocalTHCSharedAdaLNJiT:
    kwargs.setdefault("pool_groups", 768)
    return SharedReadLocalTHCSharedAdaLNJiT(
        patch_size=4, hidden_size=768, depth=12, num_heads=12, bottleneck_dim=128, workspace_grid=16, **kwargs
    )


LocalTHC_JiT_models = {
    "SharedRead-FusedFinal12-LocalTHC-SharedAdaLN-JiT-B/4": SharedRead_FusedFinal12_LocalTHC_SharedAdaLN_JiT_B_4,
    "SharedWrite-FusedFinal12-LocalTHC-SharedAdaLN-JiT-B/4": SharedRead_FusedFinal12_LocalTHC_SharedAdaLN_JiT_B_4,
    "SharedRead-FusedFinal-LocalTHC-SharedAdaLN-JiT-B/4": SharedRead_FusedFinal_LocalTHC_SharedAdaLN_JiT_B_4,
    "SharedWrite-FusedFinal-LocalTHC-SharedAdaLN-JiT-B/4": SharedRead_FusedFinal_LocalTHC_SharedAdaLN_JiT_B_4,
    "SharedRead-LocalTHC-SharedAdaLN-JiT-B/4": SharedRead_LocalTHC_SharedAdaLN_JiT_B_4,
    "SharedWrite-LocalTHC-SharedAdaLN-JiT-B/4": SharedRead_LocalTHC_SharedAdaLN_JiT_B_4,
}

_SHARED_READ_NAMES = (
    "lthc_b4_velocity",
    "local_thc_jit_shared_read_fused_final12_shared_adaln_b4",
    "local_thc_jit_shared_write_fused_final12_shared_adaln_b4",
)
# registry name -> LocalTHCV2_JiT_models key (flowmatching_lthc/models/__init__.py:29-36)
_V2_NAMES = {
    "local_thc_v2_fused_final12_shared_adaln_b4": "LocalTHCv2-FusedFinal12-SharedAdaLN-JiT-B/4",
    "local_thc_v2_fused_final12_adaln_b4": "LocalTHCv2-FusedFinal12-AdaLN-JiT-B/4",
    "local_thc_v2_direct_fused_final12_shared_adaln_b4": "LocalTHCv2-Direct-FusedFinal12-SharedAdaLN-JiT-B/4",
    "local_thc_v2_direct_fused_final12_adaln_b4": "LocalTHCv2-Direct-FusedFinal12-AdaLN-JiT-B/4",
}
MODEL_NAMES = _SHARED_READ_NAMES + tuple(_V2_NAMES)


def build_model(name: str = "lthc_b4_velocity", **kwargs) -> nn.Module:
    """The registry of the public release (flowmatching_lthc/models/__init__.py:17-38): the LTHC-B/4 shared-read
    fused-final12 model under its three names, and the four v2 models (``model_v2``).  The keys of the reference's
    LocalTHC_JiT_models (local_thc.py:1801-1827) built here are taken too: the shared-read B/4 models, and the
    per-block Triton-interface and TriangularLazy B/4 models (``model_triangular``)."""
    if name in _SHARED_READ_NAMES:
        return LocalTHC_JiT_models["SharedRead-FusedFinal12-LocalTHC-SharedAdaLN-JiT-B/4"](**kwargs)
    if name in _V2_NAMES:
        from .model_v2 import LocalTHCV2_JiT_models

        return LocalTHCV2_JiT_models[_V2_NAMES[name]](**kwargs)
    if name in LocalTHC_JiT_models:
        return LocalTHC_JiT_models[name](**kwargs)
    from .model_triangular import PerBlock_JiT_models  # imported here: that module imports this one

    if name in PerBlock_JiT_models:
        return PerBlock_JiT_models[name](**kwargs)
    available = MODEL_NAMES + tuple(LocalTHC_JiT_models) + tuple(PerBlock_JiT_models)
    raise ValueError(f"unknown model: {name}; available={available}")


@torch.no_grad()
def randomize_parameters(model: nn.Module, seed: int = 0, std: float = 0.02) -> nn.Module:
    """Re-draw every parameter (the default init zeroes the AdaLN heads and the decoder, making the output 0).

    Norm weights are drawn around 1 and the read logits around 0; everything
    else is N(0, std^2).  The draw uses one CPU generator in parameter order.
    """
    gen = torch.Generator().manual_seed(seed)
    for name, p in model.named_parameters():
        r = torch.randn(p.shape, generator=gen)
        if "norm" in name.split(".")[-2]:
            r = 1.0 + 0.1 * r
        elif name.endswith("write_weight"):
            r = 1.0 + 0.5 * r
        elif name.endswith("read_logits"):
            r = 0.5 * r
        else:
            r = std * r
        p.copy_(r.to(p.device, p.dtype))
    return model
