"""LocalTHC v2 models on the HIP interface (flowmatching_lthc/models/lthc_v2/model.py).

v2 drops the shared read: every block owns a read weight alpha_l and a write weight beta_l (plain per-channel
linear weights, no softmax), and the workspace input of block l is

    z_l = R_l(x0) + sum_{j<l} gamma[l, j] * dz_j,   gamma[l, j, c] = sum_k alpha_l[c,k] beta_j[c,k],

with X_L = x0 + sum_l P_l(dz_l) materialised once before the decoder (lthc_v2/model.py:1-12, 253-268).  The bases
R_l(x0) are the multi-weight read (``jit_thc::all_base_b4_12_split_traceable``), the sums the active-prefix
triangular ops and the materialisation ``jit_thc::final_accumulate_b4_12_traceable``, all on the gfx950 library.
Module names, constructor arguments, hooks (``_branch_update``, ``_final_accumulate``, ``_dense_output``) and
parameter names are the reference's, so its v2 checkpoints load unchanged.
"""

from __future__ import annotations

from contextlib import nullcontext

import torch
import torch.nn as nn

from . import ops
from . import ops_triangular as T
from .local_thc import overridden
from .model import (
    BatchedWeightCast,
    BottleneckPatchEmbedNHWC,
    CastLinear,
    DirectPatchEmbedNHWC,
    FinalLayer,
    FinalLayerSharedAdaLN,
    LabelEmbedder,
    TimestepEmbedder,
    VisionRotaryEmbeddingFast,
    WorkspaceJiTBranch,
    WorkspaceSharedAdaLNBranch,
    decode_output,
    materialise_decode_output,
)


class LinearChannelwisePool(nn.Module):
    """One block's read and write weights over the 16 taps of a 4x4 cell (lthc_v2/model.py:38-67):
    ``read_weight`` [C,16] (init 1/16) and ``write_weight`` [C,16] (init 1), used as they are."""

    def __init__(
        self,
        high_grid: int,
        workspace_grid: int,
        hidden_size: int,
        read_init: float | None = None,
        write_init: float = 1.0,
    ) -> None:
        super().__init__()
        if high_grid != 64 or workspace_grid != 16:
            raise ValueError("v2 fused B/4 path currently requires high_grid=64 and workspace_grid=16")
        self.high_grid = high_grid
        self.workspace_grid = workspace_grid
        self.hidden_size = hidden_size
        self.cell_size = high_grid // workspace_grid
        self.cell_tokens = self.cell_size * self.cell_size
        if self.cell_tokens != 16:
            raise ValueError(f"expected 16 local cell tokens, got {self.cell_tokens}")
        read = 1.0 / self.cell_tokens if read_init is None else float(read_init)
        self.read_weight = nn.Parameter(torch.full((hidden_size, self.cell_tokens), read))
        self.write_weight = nn.Parameter(torch.full((hidden_size, self.cell_tokens), float(write_init)))

    def alpha(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        return self.read_weight if dtype is None else self.read_weight.to(dtype=dtype)

    def beta(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        return self.write_weight if dtype is None else self.write_weight.to(dtype=dtype)


class LocalTHCV2SharedAdaLNBlock(nn.Module):
    """A v2 block: its pool weights and a shared-AdaLN workspace branch (lthc_v2/model.py:70-96)."""

    def __init__(
        self,
        hidden_size: int,
        num_heads: int,
        high_grid: int,
        workspace_grid: int = 16,
        mlp_ratio: float = 4.0,
        attn_drop: float = 0.0,
        proj_drop: float = 0.0,
        attn_backend: str = "flash",
    ) -> None:
        super().__init__()
        self.pool = LinearChannelwisePool(high_grid, workspace_grid, hidden_size)
        self.branch = WorkspaceSharedAdaLNBranch(hidden_size, num_heads, mlp_ratio, attn_drop, proj_drop, attn_backend)

    def branch_update(self, z: torch.Tensor, t6: torch.Tensor, rope: VisionRotaryEmbeddingFast) -> torch.Tensor:
        return self.branch(z, t6, rope)


class LocalTHCV2AdaLNBlock(nn.Module):
    """A v2 block whose branch has its own AdaLN head (lthc_v2/model.py:99-125)."""

    def __init__(
        self,
        hidden_size: int,
        num_heads: int,
        high_grid: int,
        workspace_grid: int = 16,
        mlp_ratio: float = 4.0,
        attn_drop: float = 0.0,
        proj_drop: float = 0.0,
        attn_backend: str = "flash",
    ) -> None:
        super().__init__()
        self.pool = LinearChannelwisePool(high_grid, workspace_grid, hidden_size)
        self.branch = WorkspaceJiTBranch(hidden_size, num_heads, mlp_ratio, attn_drop, proj_drop, attn_backend)

    def branch_update(self, z: torch.Tensor, c: torch.Tensor, rope: VisionRotaryEmbeddingFast) -> torch.Tensor:
        return self.branch(z, c, rope)


class _LocalTHCV2Base(BatchedWeightCast, nn.Module):
    """The v2 B/4 model around the non-shared lazy schedule (lthc_v2/model.py:128-271).

    Inference on the GPU takes this package's fused forms where they apply, with the hooks below left as they are:
    every linear weight converted in one launch under autocast, and the materialisation fused with the decoder
    (X_L never written; ``fused_materialise_decoder``) or the decoder as one pass (``fused_decoder``).
    """

    fused_decoder = True
    fused_materialise_decoder = True

    block_cls: type[nn.Module]
    final_cls: type[nn.Module]
    x_embedder_cls: type[nn.Module] = BottleneckPatchEmbedNHWC

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
        if input_size != 256 or patch_size != 4 or workspace_grid != 16 or depth != 12:
            raise ValueError("LocalTHC v2 fused kernel currently supports only B/4: input=256, patch=4, grid=16, depth=12")
        if pool_groups not in (None, hidden_size):
            raise ValueError("LocalTHC v2 uses per-channel pools; pool_groups must be None or hidden_size")
        self.input_size = input_size
        self.patch_size = patch_size
        self.in_channels = in_channels
        self.out_channels = in_channels
        self.hidden_size = hidden_size
        self.depth = depth
        self.num_heads = num_heads
        self.num_classes = num_classes
        self.workspace_grid = workspace_grid
        self.high_grid = input_size // patch_size
        self.num_high_tokens = self.high_grid * self.high_grid
        self.num_workspace_tokens = workspace_grid * workspace_grid
        self.pool_groups = hidden_size

        self.t_embedder = TimestepEmbedder(hidden_size)
        self.y_embedder = LabelEmbedder(num_classes, hidden_size)
        self.x_embedder = self.x_embedder_cls(input_size, patch_size, in_channels, bottleneck_dim, hidden_size)
        self.workspace_rope = VisionRotaryEmbeddingFast(hidden_size // num_heads // 2, workspace_grid, num_prefix_tokens=0)
        quarter = depth // 4
        self.blocks = nn.ModuleList(
            self.block_cls(
                hidden_size=hidden_size,
                num_heads=num_heads,
                high_grid=self.high_grid,
                workspace_grid=workspace_grid,
                mlp_ratio=mlp_ratio,
                attn_drop=attn_drop if quarter <= i < 3 * quarter else 0.0,
                proj_drop=proj_drop if quarter <= i < 3 * quarter else 0.0,
                attn_backend=attn_backend,
            )
            for i in range(depth)
        )
        self.final_layer = self.final_cls(hidden_size, patch_size, self.out_channels)
        self.initialize_weights()

    def initialize_weights(self) -> None:
        """Xavier linears with zero biases, N(0, 0.02) embeddings, zeroed AdaLN heads and decoder
        (lthc_v2/model.py:194-224)."""
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
        self._init_adaln()
        nn.init.zeros_(self.final_layer.linear.weight)
        nn.init.zeros_(self.final_layer.linear.bias)

    def _init_adaln(self) -> None:
        heads = [blk.branch.adaLN_modulation[-1] for blk in self.blocks if hasattr(blk.branch, "adaLN_modulation")]
        if hasattr(self.final_layer, "adaLN_modulation"):
            heads.append(self.final_layer.adaLN_modulation[-1])
        for head in heads:
            nn.init.zeros_(head.weight)
            nn.init.zeros_(head.bias)

    def unpatchify(self, x: torch.Tensor) -> torch.Tensor:
        """[B, h*w, p*p*c] patch rows -> [B, c, h*p, w*p] (lthc_v2/model.py:226-234)."""
        c, p = self.out_channels, self.patch_size
        h = w = int(x.shape[1] ** 0.5)
        if h * w != x.shape[1]:
            raise ValueError(f"token count {x.shape[1]} is not square")
        return x.reshape(x.shape[0], h, w, p, p, c).permute(0, 5, 1, 3, 2, 4).reshape(x.shape[0], c, h * p, w * p)

    def _pool_stack(self, hook: str, dtype: torch.dtype) -> torch.Tensor:
        """[L, C, 16] of every block's pool.alpha(dtype) or pool.beta(dtype).  Where no pool replaces the hook, the
        parameters are stacked and converted once (the values of converting each; one launch instead of 12)."""
        if any(overridden(blk.pool, hook, LinearChannelwisePool) for blk in self.blocks):
            return torch.stack([getattr(blk.pool, hook)(dtype=dtype) for blk in self.blocks]).contiguous()
        name = "read_weight" if hook == "alpha" else "write_weight"
        return torch.stack([getattr(blk.pool, name) for blk in self.blocks]).to(dtype=dtype)

    def _alpha_stack(self, dtype: torch.dtype) -> torch.Tensor:
        return self._pool_stack("alpha", dtype)

    def _beta_stack(self, dtype: torch.dtype) -> torch.Tensor:
        return self._pool_stack("beta", dtype)

    def _final_accumulate(self, x0: torch.Tensor, dz_list: list[torch.Tensor]) -> torch.Tensor:
        """X_L = x0 + sum_l P_l(dz_l), the write weights in dz's dtype (lthc_v2/model.py:242-246)."""
        if len(dz_list) != 12:
            raise ValueError("LocalTHC v2 fused final accumulation requires exactly 12 dz tensors")
        betas = list(self._pool_stack("beta", dz_list[0].dtype).unbind(0))
        return ops.final_accumulate_b4_12_traceable(x0, *dz_list, *betas)

    def _dense_output(self, x_hi: torch.Tensor, final_cond: torch.Tensor) -> torch.Tensor:
        """unpatchify(final_layer(X_L, final_cond)) (lthc_v2/model.py:248-251), one decoder pass where it applies."""
        return decode_output(self, x_hi, final_cond)

    def _run_fused_schedule(self, x0: torch.Tensor, cond: torch.Tensor) -> torch.Tensor:
        """X_L after the schedule's updates (lthc_v2/model.py:253-268)."""
        return self._final_accumulate(x0, self._schedule_updates(x0, cond))

    def _output(self, x0: torch.Tensor, cond: torch.Tensor, final_cond: torch.Tensor) -> torch.Tensor:
        """_dense_output(_run_fused_schedule(x0, cond), final_cond); with none of the three hooks replaced, the
        materialisation and the decoder in one pass where that applies."""
        if any(overridden(self, h, _LocalTHCV2Base) for h in ("_run_fused_schedule", "_final_accumulate", "_dense_output")):
            return self._dense_output(self._run_fused_schedule(x0, cond), final_cond)
        dzs = self._schedule_updates(x0, cond)
        betas = list(self._pool_stack("beta", dzs[0].dtype).unbind(0))
        out = materialise_decode_output(self, x0, dzs, betas, final_cond)
        return out if out is not None else self._dense_output(self._final_accumulate(x0, dzs), final_cond)

    def _schedule_updates(self, x0: torch.Tensor, cond: torch.Tensor) -> list[torch.Tensor]:
        """For l = 0..11: z_l = R_l(x0) + sum_{j<l} gamma[l, j] dz_j (the active-prefix op of width l, the
        unused dz slots filled with zeros), dz_l = the block's branch on z_l; returns the dz_l.
        alpha, beta and gamma are in x0's dtype, as the reference casts them."""
        alphas = self._alpha_stack(dtype=x0.dtype)
        betas = self._beta_stack(dtype=x0.dtype)
        bases = T.all_base_b4_12_split_traceable(x0, alphas)
        gamma = T.gamma_matrix(alphas, betas)
        zero_dz = torch.zeros_like(bases[0])
        dzs: list[torch.Tensor] = []
        for l, blk in enumerate(self.blocks):
            z = bases[l]
            if dzs:
                slots = tuple(dzs[j] if j < l else zero_dz for j in range(12))
                z = T.triangular_accumulate_b4_12_ptr_active_traceable_ops[l - 1](z, *slots, gamma[l].contiguous())
            dzs.append(self._branch_update(blk, z, cond))
        return dzs

    def _converted(self):
        """The one-launch weight conversion, outside torch.compile (which fuses autocast's conversions itself)."""
        return nullcontext() if torch.compiler.is_compiling() else self._converted_weights()

    def _branch_update(self, block: nn.Module, z: torch.Tensor, cond: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError


class LocalTHCV2FusedFinal12SharedAdaLNJiT(_LocalTHCV2Base):
    """v2 with one shared AdaLN head for every block and one for the decoder (lthc_v2/model.py:274-297)."""

    block_cls = LocalTHCV2SharedAdaLNBlock
    final_cls = FinalLayerSharedAdaLN

    def __init__(self, *args, **kwargs) -> None:
        super().__init__(*args, **kwargs)
        self.shared_adaLN_modulation = nn.Sequential(nn.SiLU(), CastLinear(self.hidden_size, 6 * self.hidden_size, bias=True))
        self.shared_final_modulation = nn.Sequential(nn.SiLU(), CastLinear(self.hidden_size, 2 * self.hidden_size, bias=True))
        for head in (self.shared_adaLN_modulation[-1], self.shared_final_modulation[-1]):
            nn.init.zeros_(head.weight)
            nn.init.zeros_(head.bias)

    def _branch_update(self, block: nn.Module, z: torch.Tensor, cond: torch.Tensor) -> torch.Tensor:
        return block.branch_update(z, cond, self.workspace_rope)

    def forward(self, x: torch.Tensor, t: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        with self._converted():
            c = self.t_embedder(t) + self.y_embedder(y)
            t6 = self.shared_adaLN_modulation(c)
            t2 = self.shared_final_modulation(c)
            return self._output(self.x_embedder(x), t6, t2)


class LocalTHCV2FusedFinal12AdaLNJiT(_LocalTHCV2Base):
    """v2 with an AdaLN head per block and one in the decoder (lthc_v2/model.py:300-313)."""

    block_cls = LocalTHCV2AdaLNBlock
    final_cls = FinalLayer

    def _branch_update(self, block: nn.Module, z: torch.Tensor, cond: torch.Tensor) -> torch.Tensor:
        return block.branch_update(z, cond, self.workspace_rope)

    def forward(self, x: torch.Tensor, t: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        with self._converted():
            c = self.t_embedder(t) + self.y_embedder(y)
            return self._output(self.x_embedder(x), c, c)


class LocalTHCV2DirectFusedFinal12SharedAdaLNJiT(LocalTHCV2FusedFinal12SharedAdaLNJiT):
    """The shared-AdaLN v2 with the one-GEMM patch embedding (lthc_v2/model.py:316-317)."""

    x_embedder_cls = DirectPatchEmbedNHWC


class LocalTHCV2DirectFusedFinal12AdaLNJiT(LocalTHCV2FusedFinal12AdaLNJiT):
    """The per-block AdaLN v2 with the one-GEMM patch embedding (lthc_v2/model.py:320-321)."""

    x_embedder_cls = DirectPatchEmbedNHWC


_B4 = dict(patch_size=4, hidden_size=768, depth=12, num_heads=12, bottleneck_dim=128, workspace_grid=16)


def LocalTHCV2_FusedFinal12_SharedAdaLN_JiT_B_4(**kwargs) -> LocalTHCV2FusedFinal12SharedAdaLNJiT:
    return LocalTHCV2FusedFinal12SharedAdaLNJiT(**_B4, **kwargs)


def LocalTHCV2_FusedFinal12_AdaLN_JiT_B_4(**kwargs) -> LocalTHCV2FusedFinal12AdaLNJiT:
    return LocalTHCV2FusedFinal12AdaLNJiT(**_B4, **kwargs)


def LocalTHCV2_Direct_FusedFinal12_SharedAdaLN_JiT_B_4(**kwargs) -> LocalTHCV2DirectFusedFinal12SharedAdaLNJiT:
    return LocalTHCV2DirectFusedFinal12SharedAdaLNJiT(**_B4, **kwargs)


def LocalTHCV2_Direct_FusedFinal12_AdaLN_JiT_B_4(**kwargs) -> LocalTHCV2DirectFusedFinal12AdaLNJiT:
    return LocalTHCV2DirectFusedFinal12AdaLNJiT(**_B4, **kwargs)


LocalTHCV2_JiT_models = {
    "LocalTHCv2-FusedFinal12-SharedAdaLN-JiT-B/4": LocalTHCV2_FusedFinal12_SharedAdaLN_JiT_B_4,
    "LocalTHCv2-FusedFinal12-AdaLN-JiT-B/4": LocalTHCV2_FusedFinal12_AdaLN_JiT_B_4,
    "LocalTHCv2-Direct-FusedFinal12-SharedAdaLN-JiT-B/4": LocalTHCV2_Direct_FusedFinal12_SharedAdaLN_JiT_B_4,
    "LocalTHCv2-Direct-FusedFinal12-AdaLN-JiT-B/4": LocalTHCV2_Direct_FusedFinal12_AdaLN_JiT_B_4,
}
