"""LTHC interface modules with the reference's hooks and parameter names.

Mirrors ``SharedLocalRead`` and ``LayerLocalWrite`` of
flowmatching_lthc/models/local_thc.py:1166-1283: same constructor arguments,
validation messages, parameter names (``read_logits``, ``write_weight``) and
initial values, same hook methods.  The high-resolution work (read, write,
write_add) runs through the ``jit_thc`` HIP ops of :mod:`.ops`; the [C,16]
weight math (softmax, gamma) stays in torch, as in the reference.

When ``pool_groups < hidden_size`` the per-group weights are expanded to
per-channel weights with ``repeat_interleave`` before the op, which autograd
folds back to the groups; the released model uses ``pool_groups ==
hidden_size``.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops


def _per_channel(w: torch.Tensor, group_dim: int) -> torch.Tensor:
    return w if group_dim == 1 else w.repeat_interleave(group_dim, dim=0)


class SharedLocalRead(nn.Module):
    """Depth-shared local read [B,Hh,Hh,C] -> [B,Gw*Gw,C] (local_thc.py:1166-1226)."""

    def __init__(
        self,
        high_grid: int,
        workspace_grid: int,
        hidden_size: int,
        pool_groups: int,
        use_softmax_write: bool = True,
    ) -> None:
        super().__init__()
        if high_grid % workspace_grid != 0:
            raise ValueError(f"high_grid={high_grid} must be divisible by workspace_grid={workspace_grid}")
        if hidden_size % pool_groups != 0:
            raise ValueError(f"hidden_size={hidden_size} must be divisible by pool_groups={pool_groups}")
        self.high_grid = high_grid
        self.workspace_grid = workspace_grid
        self.hidden_size = hidden_size
        self.pool_groups = pool_groups
        self.group_dim = hidden_size // pool_groups
        self.cell_size = high_grid // workspace_grid
        self.cell_tokens = self.cell_size * self.cell_size
        self.use_softmax_write = use_softmax_write
        self.read_logits = nn.Parameter(torch.zeros(pool_groups, self.cell_tokens))
        self.reset_parameters()

    def reset_parameters(self) -> None:
        nn.init.constant_(self.read_logits, 0.0)

    def alpha(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        """softmax(read_logits) in fp32 over the taps (local_thc.py:1204-1209)."""
        if self.use_softmax_write:
            alpha = F.softmax(self.read_logits.float(), dim=-1)
        else:
            alpha = self.read_logits
        return alpha if dtype is None else alpha.to(dtype=dtype)

    def read(self, x: torch.Tensor) -> torch.Tensor:
        b, h, w, c = x.shape
        hh = self.high_grid
        if h != hh or w != hh or c != self.hidden_size:
            raise ValueError(f"expected [B,{hh},{hh},{self.hidden_size}], got {tuple(x.shape)}")
        alpha = _per_channel(self.alpha(dtype=x.dtype), self.group_dim)
        return ops.local_write_traceable(x, alpha)

    def read_with_residual(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(x, read(x)) for the lazy forward, where x is read once here and materialised into at the end;
        the backward returns dX = g_x + R^T(gZ0) in one pass (ops.read_with_residual)."""
        b, h, w, c = x.shape
        hh = self.high_grid
        if h != hh or w != hh or c != self.hidden_size:
            raise ValueError(f"expected [B,{hh},{hh},{self.hidden_size}], got {tuple(x.shape)}")
        alpha = _per_channel(self.alpha(dtype=x.dtype), self.group_dim)
        return ops.read_with_residual(x, alpha)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.read(x)


class LayerLocalWrite(nn.Module):
    """Layer-specific local write [B,Gw*Gw,C] -> [B,Hh,Hh,C] (local_thc.py:1229-1283)."""

    def __init__(
        self,
        high_grid: int,
        workspace_grid: int,
        hidden_size: int,
        pool_groups: int,
        init_read: float = 1.0,
    ) -> None:
        super().__init__()
        if high_grid % workspace_grid != 0:
            raise ValueError(f"high_grid={high_grid} must be divisible by workspace_grid={workspace_grid}")
        if hidden_size % pool_groups != 0:
            raise ValueError(f"hidden_size={hidden_size} must be divisible by pool_groups={pool_groups}")
        self.high_grid = high_grid
        self.workspace_grid = workspace_grid
        self.hidden_size = hidden_size
        self.pool_groups = pool_groups
        self.group_dim = hidden_size // pool_groups
        self.cell_size = high_grid // workspace_grid
        self.cell_tokens = self.cell_size * self.cell_size
        self.write_weight = nn.Parameter(torch.full((pool_groups, self.cell_tokens), float(init_read)))
        self.reset_parameters()

    def reset_parameters(self) -> None:
        nn.init.constant_(self.write_weight, 1.0)

    def beta(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        return self.write_weight if dtype is None else self.write_weight.to(dtype=dtype)

    def channel_beta(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        """beta expanded to one row per channel, [hidden_size, cell_tokens]."""
        return _per_channel(self.beta(dtype=dtype), self.group_dim)

    def _check_dz(self, dz: torch.Tensor) -> None:
        _, n, c = dz.shape
        gw = self.workspace_grid
        if n != gw * gw or c != self.hidden_size:
            raise ValueError(f"expected [B,{gw * gw},{self.hidden_size}], got {tuple(dz.shape)}")

    def write(self, dz: torch.Tensor) -> torch.Tensor:
        self._check_dz(dz)
        return ops.local_read_traceable(dz, self.channel_beta(dtype=dz.dtype))

    def write_add(self, x_hi: torch.Tensor, dz: torch.Tensor) -> torch.Tensor:
        """x_hi + write(dz) in one pass (the stacked materialise op with L = 1)."""
        self._check_dz(dz)
        return ops.final_accumulate_b4_traceable(x_hi, dz.unsqueeze(0), self.channel_beta(dtype=dz.dtype).unsqueeze(0))

    def gamma_from_alpha(self, alpha: torch.Tensor) -> torch.Tensor:
        """gamma[c] = sum_k alpha[c,k] beta[c,k] in alpha's dtype (local_thc.py:1278-1283)."""
        beta = self.beta(dtype=alpha.dtype)
        gamma_g = (alpha * beta).sum(dim=-1)
        if self.group_dim == 1:
            return gamma_g
        return gamma_g[:, None].expand(self.pool_groups, self.group_dim).reshape(self.hidden_size)


# Backward-compatible aliases (local_thc.py:1426-1427).
SharedLocalWrite = SharedLocalRead
LayerLocalRead = LayerLocalWrite
