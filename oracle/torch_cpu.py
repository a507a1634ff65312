"""The reference's eager PyTorch op sequence for the LTHC interface, on CPU tensors.

TEST INFRASTRUCTURE ONLY.  ``bench.py``'s ``cpu_baseline`` leg times it as the
CPU baseline and ``tests/test_oracle.py`` pins it against the numpy oracle;
the product path never imports it.

Each function restates one reference method as the same tensor operations
(views, permutes, broadcast multiplies, sums) in the same order, so the work a
CPU does for the reference's own path is what is timed:

* ``read``        -- ``SharedLocalRead.read``, local_thc.py:1211-1223
* ``gamma``       -- ``LayerLocalWrite.gamma_from_alpha``, local_thc.py:1278-1283
* ``recur``       -- ``SharedReadLocalTHCSharedAdaLNJiTBlock.lazy_workspace_update``, local_thc.py:1325-1328
* ``write_add``   -- ``LayerLocalWrite.write`` + ``write_add``, local_thc.py:1261-1276
* ``materialise`` -- ``final_accumulate_reference``, the write_add loop, local_thc.py:1368-1372
* ``step``        -- the interface part of ``forward_lazy`` (local_thc.py:1376-1394) with the branch
  outputs dZ_l given: read once, L recurrence steps, one materialisation.

Channel-wise weights (pool_groups == C, group_dim == 1) as in the released model.
"""

from __future__ import annotations

import torch

S = 4  # cell side


def read(x: torch.Tensor, alpha: torch.Tensor, G: int) -> torch.Tensor:
    """[B, 4G, 4G, C] -> [B, G*G, C]: z = sum over the cell's taps of x * alpha (local_thc.py:1218-1223)."""
    b, _, _, c = x.shape
    xv = x.view(b, G, S, G, S, c, 1)
    a = alpha.to(x.dtype).view(c, S, S).permute(1, 2, 0)
    z = (xv * a[None, None, :, None, :, :, None]).sum(dim=(2, 4))
    return z.reshape(b, G * G, c)


def gamma(alpha: torch.Tensor, beta: torch.Tensor) -> torch.Tensor:
    """gamma[c] = sum_k alpha[c,k] beta[c,k] in alpha's dtype (local_thc.py:1278-1283)."""
    return (alpha * beta.to(alpha.dtype)).sum(dim=-1)


def recur(z: torch.Tensor, dz: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """Z_{l+1} = Z_l + gamma[None, None, :] * dZ_l (local_thc.py:1325-1328)."""
    return z + g[None, None, :] * dz


def write_add(x_hi: torch.Tensor, dz: torch.Tensor, beta: torch.Tensor, G: int) -> torch.Tensor:
    """x_hi + P(dz): every tap of a cell gets beta[c,k] * dz[cell, c] (local_thc.py:1261-1276)."""
    b, _, c = dz.shape
    dzv = dz.view(b, G, G, c, 1)
    bt = beta.to(dz.dtype).view(c, S, S).permute(1, 2, 0)
    dx = dzv[:, :, None, :, None, :, :] * bt[None, None, :, None, :, :, None]
    return x_hi + dx.reshape(b, G * S, G * S, c)


def materialise(x0: torch.Tensor, dzs, betas, G: int) -> torch.Tensor:
    """X_L = X_0 + sum_l P_l(dZ_l) as the reference's write_add loop (local_thc.py:1368-1372)."""
    x = x0
    for dz, bt in zip(dzs, betas, strict=True):
        x = write_add(x, dz, bt, G)
    return x


def step(x0: torch.Tensor, alpha: torch.Tensor, betas, dzs, G: int):
    """One interface forward with the branch outputs given: Z_0 = R(X_0), Z_{l+1} = Z_l + gamma_l dZ_l for every
    layer, X_L = X_0 + sum_l P_l(dZ_l).  Returns (Z_L, X_L)."""
    z = read(x0, alpha, G)
    for dz, bt in zip(dzs, betas, strict=True):
        z = recur(z, dz, gamma(alpha.to(dz.dtype), bt))
    return z, materialise(x0, dzs, betas, G)
