"""Per-block LocalTHC models and the TriangularLazy models built on them (flowmatching_lthc/models/local_thc.py).

Per-block models (local_thc.py:759-787, :823-844, :876-1018, :1108-1153).  Every block owns a
hyper-connection ``hyper`` with a read ``read_logits`` and a write ``write_weight``, both [C,16] (the
``ChannelwiseLocalTokenHyperConnectionTriton*`` modules of :mod:`.local_thc`), and a shared-AdaLN workspace
branch.  The high-resolution stream goes through every block:

    z_l = R_l(x_l),   dz_l = branch_l(z_l),   x_{l+1} = x_l + P_l(dz_l),

with R_l the softmax-weighted read of each 4x4 cell and P_l the write back to its 16 tokens, each a ``jit_thc``
HIP op.

TriangularLazy models (local_thc.py:1434-1535).  R_l P_j acts per channel, as the scale
gamma[l, j, c] = sum_k alpha_l[c, k] beta_j[c, k], so

    z_l = R_l(x0) + sum_{j<l} gamma[l, j] * dz_j,   x_L = x0 + sum_l P_l(dz_l),

and the stream is never formed between blocks: one multi-weight read gives every R_l(x0)
(``jit_thc::all_base_b4_12_traceable``), each block's input is one active-prefix triangular sum
(``jit_thc::triangular_accumulate_b4_12_ptr_active{l}``) and x_L is materialised once
(``jit_thc::final_accumulate_b4_12_traceable``).  ``forward(..., use_lazy=False)`` runs the per-block recurrence
of the parent class instead.

Class names, constructor arguments, module tree and parameter names are the reference's, so its checkpoints load
unchanged.  The reference's Triton modules only take the 64x64 / 16x16 geometry; these take any grid whose cell
side is 4 (the TriangularLazy forward keeps the reference's depth of 12).
"""

from __future__ import annotations

from contextlib import nullcontext

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from . import ops_triangular as T
from .local_thc import (
    overridden,
    ChannelwiseLocalTokenHyperConnectionTriton,
    ChannelwiseLocalTokenHyperConnectionTritonFrozen,
    ChannelwiseLocalTokenHyperConnectionTritonReadAdd,
    ChannelwiseLocalTokenHyperConnectionTritonTraceable,
)
from .model import (
    BatchedWeightCast,
    BottleneckPatchEmbedNHWC,
    CastLinear,
    DirectPatchEmbedNHWC,
    FinalLayerSharedAdaLN,
    LabelEmbedder,
    TimestepEmbedder,
    VisionRotaryEmbeddingFast,
    WorkspaceSharedAdaLNBranch,
    decode_output,
    materialise_decode_output,
    migrate_lthc_state_dict_keys,
)


class LocalTHCTritonSharedAdaLNJiTBlock(nn.Module):
    """One block: its hyper-connection and a shared-AdaLN workspace branch (local_thc.py:759-787, :823-826)."""

    hyper_cls: type[nn.Module] = ChannelwiseLocalTokenHyperConnectionTriton

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
        self.hyper = self.hyper_cls(high_grid, workspace_grid, hidden_size, pool_groups)
        self.branch = WorkspaceSharedAdaLNBranch(hidden_size, num_heads, mlp_ratio, attn_drop, proj_drop, attn_backend)

    def forward(self, x_hi: torch.Tensor, t6: torch.Tensor, rope: VisionRotaryEmbeddingFast) -> torch.Tensor:
        """x_hi + P(branch(R(x_hi))), the write fused with the add where the hyper-connection has that form."""
        z = self.hyper.read_from_residual(x_hi)
        dz = self.branch(z, t6, rope)
        if hasattr(self.hyper, "write_to_residual_add"):
            return self.hyper.write_to_residual_add(dz, x_hi)
        return x_hi + self.hyper.write_to_residual(dz)


class LocalTHCTritonReadAddSharedAdaLNJiTBlock(LocalTHCTritonSharedAdaLNJiTBlock):
    """The write fused with the residual add (local_thc.py:829-832)."""

    hyper_cls = ChannelwiseLocalTokenHyperConnectionTritonReadAdd


class LocalTHCTritonFrozenSharedAdaLNJiTBlock(LocalTHCTritonSharedAdaLNJiTBlock):
    """Read and write-add whose weights get no gradient (local_thc.py:835-838)."""

    hyper_cls = ChannelwiseLocalTokenHyperConnectionTritonFrozen


class LocalTHCTritonTraceableSharedAdaLNJiTBlock(LocalTHCTritonSharedAdaLNJiTBlock):
    """Read and write-add through the traceable ops (local_thc.py:841-844)."""

    hyper_cls = ChannelwiseLocalTokenHyperConnectionTritonTraceable


class LocalTHCTritonSharedAdaLNJiT(BatchedWeightCast, nn.Module):
    """Per-block LocalTHC JiT with shared AdaLN heads (local_thc.py:876-1018, :1108-1111).

    Inference on the GPU takes this package's fused forms where they apply: every linear weight converted in one
    launch under autocast, and the decoder as one pass (``fused_decoder``).
    """

    block_cls: type[nn.Module] = LocalTHCTritonSharedAdaLNJiTBlock
    x_embedder_cls: type[nn.Module] = BottleneckPatchEmbedNHWC
    fused_decoder = True
    fused_materialise_decoder = True

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
        self.x_embedder = self.x_embedder_cls(input_size, patch_size, in_channels, bottleneck_dim, hidden_size)
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

    def initialize_weights(self) -> None:
        """Xavier linears and patch projections with zero biases, N(0, 0.02) embeddings, zeroed AdaLN heads and
        decoder (local_thc.py:944-970, :1004-1007); the hyper-connections keep their own initial values."""
        for m in self.modules():
            if isinstance(m, nn.Linear):
                nn.init.xavier_uniform_(m.weight)
                if m.bias is not None:
                    nn.init.zeros_(m.bias)
        emb = self.x_embedder
        convs = (emb.proj,) if hasattr(emb, "proj") else (emb.proj1, emb.proj2)
        for conv in convs:
            nn.init.xavier_uniform_(conv.weight.data.view(conv.weight.shape[0], -1))
        if convs[-1].bias is not None:
            nn.init.zeros_(convs[-1].bias)
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

    def unpatchify(self, x: torch.Tensor) -> torch.Tensor:
        """[B, h*w, p*p*c] patch rows -> [B, c, h*p, w*p] (local_thc.py:972-980)."""
        c, p = self.out_channels, self.patch_size
        h = w = int(x.shape[1] ** 0.5)
        if h * w != x.shape[1]:
            raise ValueError(f"token count {x.shape[1]} is not square")
        return x.reshape(x.shape[0], h, w, p, p, c).permute(0, 5, 1, 3, 2, 4).reshape(x.shape[0], c, h * p, w * p)

    def _conditioning(self, t: torch.Tensor, y: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        c = self.t_embedder(t) + self.y_embedder(y)
        return self.shared_adaLN_modulation(c), self.shared_final_modulation(c)

    def _dense_output(self, x_hi: torch.Tensor, t2: torch.Tensor) -> torch.Tensor:
        """unpatchify(final_layer(X, t2)), one decoder pass where it applies."""
        return decode_output(self, x_hi, t2)

    def _converted(self):
        """The one-launch weight conversion, outside torch.compile (which fuses autocast's conversions itself)."""
        return nullcontext() if torch.compiler.is_compiling() else self._converted_weights()

    def _forward_per_block(self, x: torch.Tensor, t: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        t6, t2 = self._conditioning(t, y)
        x_hi = self.x_embedder(x)
        for block in self.blocks:
            x_hi = block(x_hi, t6, self.workspace_rope)
        return self._dense_output(x_hi, t2)

    def forward(self, x: torch.Tensor, t: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        """Per-block recurrence over the high-resolution stream (local_thc.py:1009-1018)."""
        with self._converted():
            return self._forward_per_block(x, t, y)


class LocalTHCDirectTritonSharedAdaLNJiT(LocalTHCTritonSharedAdaLNJiT):
    """With the one-GEMM patch embedding (local_thc.py:1114-1117)."""

    x_embedder_cls = DirectPatchEmbedNHWC


class LocalTHCTritonReadAddSharedAdaLNJiT(LocalTHCTritonSharedAdaLNJiT):
    """Write fused with the residual add (local_thc.py:1120-1123)."""

    block_cls = LocalTHCTritonReadAddSharedAdaLNJiTBlock


class LocalTHCDirectTritonReadAddSharedAdaLNJiT(LocalTHCTritonReadAddSharedAdaLNJiT):
    """local_thc.py:1126-1129."""

    x_embedder_cls = DirectPatchEmbedNHWC


class LocalTHCTritonFrozenSharedAdaLNJiT(LocalTHCTritonSharedAdaLNJiT):
    """Hyper-connection weights without gradients (local_thc.py:1132-1135)."""

    block_cls = LocalTHCTritonFrozenSharedAdaLNJiTBlock


class LocalTHCDirectTritonFrozenSharedAdaLNJiT(LocalTHCTritonFrozenSharedAdaLNJiT):
    """local_thc.py:1138-1141."""

    x_embedder_cls = DirectPatchEmbedNHWC


class LocalTHCTritonTraceableSharedAdaLNJiT(LocalTHCTritonSharedAdaLNJiT):
    """Traceable read and write-add ops (local_thc.py:1144-1147)."""

    block_cls = LocalTHCTritonTraceableSharedAdaLNJiTBlock


class LocalTHCDirectTritonTraceableSharedAdaLNJiT(LocalTHCTritonTraceableSharedAdaLNJiT):
    """local_thc.py:1150-1153."""

    x_embedder_cls = DirectPatchEmbedNHWC


class TriangularLazyFusedFinal12LocalTHCDirectTritonSharedAdaLNJiT(LocalTHCDirectTritonTraceableSharedAdaLNJiT):
    """The per-block model run by the exact triangular lazy schedule (local_thc.py:1434-1520).

    forward_lazy: every R_l(x0) from one read of x0, z_l as an active-prefix triangular sum of the earlier
    updates, x_L materialised once.  forward_naive: the parent's per-block recurrence.  Both give the same
    values up to rounding.
    """

    def _expanded_alpha(self, block: nn.Module, dtype: torch.dtype) -> torch.Tensor:
        """The block's read weights, one row per channel: softmax(read_logits) in fp32 then cast to dtype
        (local_thc.py:1455-1465)."""
        hyper = block.hyper
        alpha = F.softmax(hyper.read_logits.float(), dim=-1) if hyper.use_softmax_write else hyper.read_logits
        alpha = alpha.to(dtype=dtype)
        if hyper.group_dim == 1:
            return alpha
        return alpha.repeat_interleave(hyper.group_dim, dim=0)

    def _expanded_beta(self, block: nn.Module, dtype: torch.dtype) -> torch.Tensor:
        """The block's write weights in dtype, one row per channel (local_thc.py:1467-1474)."""
        hyper = block.hyper
        beta = hyper.write_weight.to(dtype=dtype)
        if hyper.group_dim == 1:
            return beta
        return beta.repeat_interleave(hyper.group_dim, dim=0)

    def _check_depth(self, n: int) -> None:
        if n != 12 or len(self.blocks) != 12:
            raise ValueError(f"{type(self).__name__} requires depth=12")

    def final_accumulate_reference(self, x0: torch.Tensor, dz_list: list[torch.Tensor]) -> torch.Tensor:
        """x_L = x0 + sum_l P_l(dz_l) in one pass, the write weights in dz's dtype (local_thc.py:1476-1480)."""
        self._check_depth(len(dz_list))
        betas = list(self._beta_stack(dz_list[0].dtype).unbind(0))
        return ops.final_accumulate_b4_12_traceable(x0, *dz_list, *betas)

    def forward_naive(self, x: torch.Tensor, t: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        """The per-block recurrence (local_thc.py:1482-1484)."""
        with self._converted():
            return self._forward_per_block(x, t, y)

    def _simple_hyper(self, hook: str) -> bool:
        """The hook is the class's own and every block has one pool group per channel and softmax read weights: the
        stack of its results is one operation over the stacked parameters."""
        base = TriangularLazyFusedFinal12LocalTHCDirectTritonSharedAdaLNJiT
        return not overridden(self, hook, base) and all(
            blk.hyper.group_dim == 1 and blk.hyper.use_softmax_write for blk in self.blocks
        )

    def _alpha_stack(self, dtype: torch.dtype) -> torch.Tensor:
        """[L, C, 16] of _expanded_alpha in dtype: one softmax over the stacked logits where that hook is the class's
        own (the softmax is per row, so the values are the same; a stack, a softmax and a conversion instead of one
        of each per block)."""
        if self._simple_hyper("_expanded_alpha"):
            logits = torch.stack([blk.hyper.read_logits for blk in self.blocks], dim=0)
            return F.softmax(logits.float(), dim=-1).to(dtype=dtype)
        return torch.stack([self._expanded_alpha(blk, dtype) for blk in self.blocks], dim=0)

    def _beta_stack(self, dtype: torch.dtype) -> torch.Tensor:
        """[L, C, 16] of _expanded_beta in dtype: one conversion of the stacked parameters where that hook is the
        class's own."""
        if self._simple_hyper("_expanded_beta"):
            return torch.stack([blk.hyper.write_weight for blk in self.blocks], dim=0).to(dtype=dtype)
        return torch.stack([self._expanded_beta(blk, dtype) for blk in self.blocks], dim=0)

    def forward_lazy(self, x: torch.Tensor, t: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        """local_thc.py:1486-1515.  alpha, beta and gamma are in x0's dtype, as the reference casts them; the unused
        slots of each active-prefix sum hold one zero tensor.  With final_accumulate_reference and _dense_output
        as they are, inference on the GPU materialises x_L inside the decoder's pass (never written)."""
        self._check_depth(len(self.blocks))
        with self._converted():
            return self._forward_lazy(x, t, y)

    def _forward_lazy(self, x: torch.Tensor, t: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        t6, t2 = self._conditioning(t, y)
        x0 = self.x_embedder(x)
        alpha_stack, beta_stack = self._alpha_stack(x0.dtype), self._beta_stack(x0.dtype)
        base_stack = T.all_base_b4_12_traceable(x0, alpha_stack.contiguous())
        gamma = T.gamma_matrix(alpha_stack, beta_stack)
        zero_dz = torch.zeros_like(base_stack[0])
        dz_list: list[torch.Tensor] = []
        for l, block in enumerate(self.blocks):
            z = base_stack[l]
            if dz_list:
                slots = tuple(dz_list[j] if j < l else zero_dz for j in range(12))
                z = T.triangular_accumulate_b4_12_ptr_active_traceable_ops[l - 1](z, *slots, gamma[l].contiguous())
            dz_list.append(block.branch(z, t6, self.workspace_rope))
        base = TriangularLazyFusedFinal12LocalTHCDirectTritonSharedAdaLNJiT
        if not any(overridden(self, h, base) for h in ("final_accumulate_reference", "_dense_output", "_expanded_beta")):
            out = materialise_decode_output(self, x0, dz_list, list(beta_stack.unbind(0)), t2)
            if out is not None:
                return out
        return self._dense_output(self.final_accumulate_reference(x0, dz_list), t2)

    def forward(self, x: torch.Tensor, t: torch.Tensor, y: torch.Tensor, use_lazy: bool = True) -> torch.Tensor:
        return self.forward_lazy(x, t, y) if use_lazy else self.forward_naive(x, t, y)


class TriangularLazyFusedFinal12LocalTHCTritonTraceableSharedAdaLNJiT(
    TriangularLazyFusedFinal12LocalTHCDirectTritonSharedAdaLNJiT
):
    """The B/4 LocalTHC architecture with the two-stage bottleneck patch embedding, run by the triangular lazy
    schedule (local_thc.py:1523-1534)."""

    x_embedder_cls = BottleneckPatchEmbedNHWC


_B4 = dict(patch_size=4, hidden_size=768, depth=12, num_heads=12, bottleneck_dim=128, workspace_grid=16)


def _b4(cls: type[nn.Module]):
    """The B/4 registry constructor of cls (local_thc.py:1625-1648, :1722-1749): pool_groups defaults to 768."""

    def build(**kwargs) -> nn.Module:
        kwargs.setdefault("pool_groups", 768)
        return cls(**_B4, **kwargs)

    build.__name__ = build.__qualname__ = f"{cls.__name__}_B_4"
    return build


LocalTHC_Triton_SharedAdaLN_JiT_B_4 = _b4(LocalTHCTritonSharedAdaLNJiT)
LocalTHC_Direct_Triton_SharedAdaLN_JiT_B_4 = _b4(LocalTHCDirectTritonSharedAdaLNJiT)
LocalTHC_Direct_Triton_ReadAdd_SharedAdaLN_JiT_B_4 = _b4(LocalTHCDirectTritonReadAddSharedAdaLNJiT)
LocalTHC_Direct_Triton_Frozen_SharedAdaLN_JiT_B_4 = _b4(LocalTHCDirectTritonFrozenSharedAdaLNJiT)
LocalTHC_Direct_Triton_Traceable_SharedAdaLN_JiT_B_4 = _b4(LocalTHCDirectTritonTraceableSharedAdaLNJiT)
TriangularLazy_FusedFinal12_LocalTHC_DirectTriton_SharedAdaLN_JiT_B_4 = _b4(
    TriangularLazyFusedFinal12LocalTHCDirectTritonSharedAdaLNJiT
)
TriangularLazy_FusedFinal12_LocalTHC_TritonTraceable_SharedAdaLN_JiT_B_4 = _b4(
    TriangularLazyFusedFinal12LocalTHCTritonTraceableSharedAdaLNJiT
)

# Registry entries (local_thc.py:1801-1827) of the models in this module.
PerBlock_JiT_models = {
    "LocalTHC-Triton-SharedAdaLN-JiT-B/4": LocalTHC_Triton_SharedAdaLN_JiT_B_4,
    "LocalTHC-Direct-Triton-SharedAdaLN-JiT-B/4": LocalTHC_Direct_Triton_SharedAdaLN_JiT_B_4,
    "LocalTHC-Direct-Triton-ReadAdd-SharedAdaLN-JiT-B/4": LocalTHC_Direct_Triton_ReadAdd_SharedAdaLN_JiT_B_4,
    "LocalTHC-Direct-Triton-Frozen-SharedAdaLN-JiT-B/4": LocalTHC_Direct_Triton_Frozen_SharedAdaLN_JiT_B_4,
    "LocalTHC-Direct-Triton-Traceable-SharedAdaLN-JiT-B/4": LocalTHC_Direct_Triton_Traceable_SharedAdaLN_JiT_B_4,
    "TriangularLazy-FusedFinal12-LocalTHC-DirectTriton-SharedAdaLN-JiT-B/4": (
        TriangularLazy_FusedFinal12_LocalTHC_DirectTriton_SharedAdaLN_JiT_B_4
    ),
    "TriangularLazy-FusedFinal12-LocalTHC-TritonTraceable-SharedAdaLN-JiT-B/4": (
        TriangularLazy_FusedFinal12_LocalTHC_TritonTraceable_SharedAdaLN_JiT_B_4
    ),
}
