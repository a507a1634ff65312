"""LTHC interface modules with the reference's hooks and parameter names.

Mirrors ``SharedLocalRead`` and ``LayerLocalWrite`` of
flowmatching_lthc/models/local_thc.py:1166-1283, and the per-block
``ChannelwiseLocalTokenHyperConnectionTriton*`` modules of :511-617: same constructor arguments,
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


def overridden(obj: nn.Module, name: str, base: type) -> bool:
    """True when obj's hook `name` is not base's own: replaced on a subclass or assigned on the instance."""
    return getattr(type(obj), name, None) is not getattr(base, name) or name in obj.__dict__


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
        the backward returns dX = g_x + R^T(gZ0) in one pass (ops.read_with_residual).  A replaced `read` or
        `alpha` hook (subclass or instance) is honoured: then this is (x, self.read(x))."""
        if overridden(self, "read", SharedLocalRead) or overridden(self, "alpha", SharedLocalRead):
            return x, self.read(x)
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


class ChannelwiseLocalTokenHyperConnectionTriton(nn.Module):
    """Per-block read and write with one module (local_thc.py:511-561): ``read_logits`` and ``write_weight``
    [C,16], read = R_softmax(read_logits)(x), write = P_write_weight(dz), both with weight gradients.

    The reference's version only runs the 64x64 / 16x16 geometry; this one takes any grid whose cell side
    is 4.  It keeps the reference's other restrictions: pool_groups == hidden_size and softmax read weights.
    """

    def __init__(
        self,
        high_grid: int,
        workspace_grid: int,
        hidden_size: int,
        pool_groups: int,
        use_softmax_write: bool = True,
        init_read: float = 1.0,
    ) -> None:
        super().__init__()
        if high_grid != ops.S * workspace_grid:
            raise ValueError(f"LocalTHC HIP ops need cell side {ops.S}: high_grid={high_grid}, workspace_grid={workspace_grid}")
        if pool_groups != hidden_size:
            raise ValueError("Triton LocalTHC currently requires pool_groups == hidden_size")
        if not use_softmax_write:
            raise ValueError("Triton LocalTHC currently assumes softmax read weights")
        self.high_grid = high_grid
        self.workspace_grid = workspace_grid
        self.hidden_size = hidden_size
        self.pool_groups = pool_groups
        self.group_dim = 1
        self.cell_size = ops.S
        self.cell_tokens = ops.K
        self.use_softmax_write = use_softmax_write
        self.read_logits = nn.Parameter(torch.zeros(hidden_size, self.cell_tokens))
        self.write_weight = nn.Parameter(torch.full((hidden_size, self.cell_tokens), float(init_read)))
        self.reset_parameters()

    def reset_parameters(self) -> None:
        nn.init.constant_(self.read_logits, 0.0)
        nn.init.constant_(self.write_weight, 1.0)

    def _alpha(self, dtype: torch.dtype) -> torch.Tensor:
        return F.softmax(self.read_logits.float(), dim=-1).to(dtype=dtype)

    def read_from_residual(self, x: torch.Tensor) -> torch.Tensor:
        return ops.local_write(x, self._alpha(x.dtype))

    def write_to_residual(self, dz: torch.Tensor) -> torch.Tensor:
        return ops.local_read(dz, self.write_weight.to(dtype=dz.dtype))

    def read(self, x: torch.Tensor) -> torch.Tensor:
        return self.read_from_residual(x)

    def write(self, dz: torch.Tensor) -> torch.Tensor:
        return self.write_to_residual(dz)


class ChannelwiseLocalTokenHyperConnectionTritonReadAdd(ChannelwiseLocalTokenHyperConnectionTriton):
    """The write fused with the outer residual add, x + P(dz) in one pass (local_thc.py:564-571)."""

    def write_to_residual_add(self, dz: torch.Tensor, x_hi: torch.Tensor) -> torch.Tensor:
        return ops.local_read_add(dz, self.write_weight.to(dtype=dz.dtype), x_hi)

    def write_add(self, dz: torch.Tensor, x_hi: torch.Tensor) -> torch.Tensor:
        return self.write_to_residual_add(dz, x_hi)


class ChannelwiseLocalTokenHyperConnectionTritonFrozen(ChannelwiseLocalTokenHyperConnectionTriton):
    """Read and fused write-add whose weights get no gradient (local_thc.py:574-594)."""

    def read_from_residual(self, x: torch.Tensor) -> torch.Tensor:
        return ops.local_write_no_weight_grad(x, self._alpha(x.dtype))

    def write_to_residual_add(self, dz: torch.Tensor, x_hi: torch.Tensor) -> torch.Tensor:
        return ops.local_read_add_no_weight_grad(dz, self.write_weight.to(dtype=dz.dtype), x_hi)

    def write_to_residual(self, dz: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError("Use write_to_residual_add for TritonFrozen LocalTHC.")

    def write_add(self, dz: torch.Tensor, x_hi: torch.Tensor) -> torch.Tensor:
        return self.write_to_residual_add(dz, x_hi)


class ChannelwiseLocalTokenHyperConnectionTritonTraceable(ChannelwiseLocalTokenHyperConnectionTriton):
    """Read and fused write-add through the ``jit_thc`` ops, with weight gradients (local_thc.py:597-617)."""

    def read_from_residual(self, x: torch.Tensor) -> torch.Tensor:
        return ops.local_write_traceable(x, self._alpha(x.dtype))

    def write_to_residual_add(self, dz: torch.Tensor, x_hi: torch.Tensor) -> torch.Tensor:
        return ops.local_read_add_traceable(dz, self.write_weight.to(dtype=dz.dtype), x_hi)

    def write_to_residual(self, dz: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError("Use write_to_residual_add for TritonTraceable LocalTHC.")

    def write_add(self, dz: torch.Tensor, x_hi: torch.Tensor) -> torch.Tensor:
        return self.write_to_residual_add(dz, x_hi)


# Backward-compatible aliases (local_thc.py:1426-1427).
SharedLocalWrite = SharedLocalRead
LayerLocalRead = LayerLocalWrite
