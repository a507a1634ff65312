"""CPU oracle of the LTHC read / write / materialise interface.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg import this module, and only as the
checker or the CPU baseline.  The product path (``flowmatching_lthc_amd``)
never imports it and has no CPU fallback.

Two independent restatements of the reference algorithm live here:

* ``*_np`` — numpy, float64, written as the reference's own eager PyTorch op
  sequence (view / permute / broadcast-multiply / sum) of
  ``flowmatching_lthc/models/local_thc.py``.
* ``C*`` — a plain C restatement (``lthc_oracle.c``: explicit index map, fp64
  accumulation, OpenMP), fast enough for the benchmark shapes; it is also the
  CPU baseline that ``bench.py`` times.

How each function is pinned (tests/test_oracle.py):

=====================  ==================================================================
function               pinned by
=====================  ==================================================================
read_np / Cread        brute-force loops over the explicit index map; depthwise
                       ``F.conv2d(stride=s, groups=C)``; alpha == 1/16 -> ``avg_pool2d``
write_np / Cwrite      brute-force loops; depthwise ``F.conv_transpose2d``; beta == 1 ->
                       nearest ``repeat_interleave`` upsample; adjoint identity
                       <R X, Z> == <X, R^T Z> against read
gamma_np / Cgamma      R(P_l(dZ)) == gamma_l * dZ on random data (the exact lazy identity)
lazy recurrence        R(X0 + sum_{j<l} P_j dZ_j) == Z0 + sum_{j<l} gamma_j dZ_j for every l
final accumulate       equals the iterative write_add loop; dZ == 0 gives X0
weight_grad_np / C     ``torch.autograd`` of the reference op sequence (read and write)
read_multi / Cread_m   ``torch.autograd`` of the materialisation w.r.t. each dZ_l
interface_bwd_np       ``torch.autograd`` of the whole lazy interface (float64), and
                       ``torch.autograd.gradcheck`` of the torch restatement
recur_bwd              ``torch.autograd`` of z + gamma * dz
triangular_lazy_np     z_l == R_l(X0 + sum_{j<l} P_j dZ_j) with separate R_l / P_j per layer
(triangular_np,        (depthwise-conv reads of the naively materialised stream), for every l;
gamma_matrix_np)       gamma[l, j] == R_l P_j on random data; dropped or extra j caught
=====================  ==================================================================

Plausible mistakes (swapped sy/sx, transposed weight [K,C] vs [C,K], dropped
layer, wrong sign) each fail at least one of these checks; the mutation tests
in tests/test_oracle.py plant them in copies of these functions and assert
that the checks catch them.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "lthc_oracle.c")
LIB = os.path.join(HERE, "liblthc_oracle.so")


# ---------------------------------------------------------------------------
# Geometry helpers (index map: local_thc_triton_kernels.py:355-363)
# ---------------------------------------------------------------------------
def grid_of(h: int, m: int) -> tuple[int, int]:
    """(G, S) from the high-res side ``h`` and the workspace cell count ``m``."""
    g = math.isqrt(m)
    if g * g != m or h % g != 0:
        raise ValueError(f"cells={m} / high grid={h} do not form a square cell grid")
    return g, h // g


def to_cells(x: np.ndarray, g: int) -> np.ndarray:
    """NHWC [B,H,H,C] -> cell view [B, G*G, S*S, C]."""
    b, h, _, c = x.shape
    s = h // g
    return x.reshape(b, g, s, g, s, c).transpose(0, 1, 3, 2, 4, 5).reshape(b, g * g, s * s, c)


# ---------------------------------------------------------------------------
# numpy restatement (float64), following the reference's eager op sequence
# ---------------------------------------------------------------------------
def read_np(x: np.ndarray, alpha: np.ndarray, g: int) -> np.ndarray:
    """Z = R(X): local_thc.py:1211-1223 (view [b,gw,s,gw,s,C], alpha.view(C,s,s).permute(1,2,0), sum over (2,4))."""
    b, h, _, c = x.shape
    s = h // g
    xv = np.asarray(x, np.float64).reshape(b, g, s, g, s, c)
    a = np.asarray(alpha, np.float64).reshape(c, s, s).transpose(1, 2, 0)
    z = (xv * a[None, None, :, None, :, :]).sum(axis=(2, 4))
    return z.reshape(b, g * g, c)


def write_np(dz: np.ndarray, beta: np.ndarray, h: int) -> np.ndarray:
    """P(dZ): local_thc.py:1261-1273 (dz[:, :, None, :, None, :] * beta[None, None, :, None, :, :])."""
    b, m, c = dz.shape
    g, s = grid_of(h, m)
    dzv = np.asarray(dz, np.float64).reshape(b, g, g, c)
    be = np.asarray(beta, np.float64).reshape(c, s, s).transpose(1, 2, 0)
    dx = dzv[:, :, None, :, None, :] * be[None, None, :, None, :, :]
    return dx.reshape(b, h, h, c)


def write_add_np(x: np.ndarray, dz: np.ndarray, beta: np.ndarray) -> np.ndarray:
    """LayerLocalWrite.write_add: local_thc.py:1275-1276."""
    return np.asarray(x, np.float64) + write_np(dz, beta, x.shape[1])


def gamma_np(alpha: np.ndarray, beta: np.ndarray) -> np.ndarray:
    """gamma_from_alpha: local_thc.py:1278-1283 ((alpha * beta).sum(-1))."""
    return (np.asarray(alpha, np.float64) * np.asarray(beta, np.float64)).sum(-1)


def lazy_update_np(z: np.ndarray, dz: np.ndarray, gamma: np.ndarray) -> np.ndarray:
    """lazy_workspace_update: local_thc.py:1325-1328."""
    return np.asarray(z, np.float64) + np.asarray(gamma, np.float64)[None, None, :] * np.asarray(dz, np.float64)


def final_accumulate_np(x0: np.ndarray, dz_list, beta_list) -> np.ndarray:
    """final_accumulate_reference loop: local_thc.py:1368-1372."""
    x = np.asarray(x0, np.float64)
    for dz, beta in zip(dz_list, beta_list, strict=True):
        x = write_add_np(x, dz, beta)
    return x


def weight_grad_np(high: np.ndarray, low: np.ndarray, g: int) -> np.ndarray:
    """gw[c,k] = sum_{b,m} high[b,m,k,c] low[b,m,c] (_cell_weight_grad_kernel :167-199)."""
    hc = to_cells(np.asarray(high, np.float64), g)
    return np.einsum("bmkc,bmc->ck", hc, np.asarray(low, np.float64))


def lazy_forward_np(x0, alpha, dz_list, beta_list, g):
    """forward_lazy interface part (local_thc.py:1374-1388): Z_0..Z_L and X_L."""
    z = read_np(x0, alpha, g)
    zs = [z]
    for dz, beta in zip(dz_list, beta_list, strict=True):
        z = lazy_update_np(z, dz, gamma_np(alpha, beta))
        zs.append(z)
    return zs, final_accumulate_np(x0, dz_list, beta_list)


def gamma_matrix_np(alpha_list, beta_list) -> np.ndarray:
    """gamma[l, j, c] = sum_k alpha_l[c,k] beta_j[c,k] (local_thc.py:1496; lthc_v2/model.py:257)."""
    a = np.stack([np.asarray(x, np.float64) for x in alpha_list])
    b = np.stack([np.asarray(x, np.float64) for x in beta_list])
    return (a[:, None, :, :] * b[None, :, :, :]).sum(-1)


def triangular_np(base: np.ndarray, dz_list, gamma_rows) -> np.ndarray:
    """triangular_accumulate: base + sum_{i < len(dz_list)} gamma_rows[i] * dz_i
    (local_thc_triton_kernels.py:1922-2012; the active-prefix forms :2161-2488 use the first `active` layers)."""
    out = np.asarray(base, np.float64).copy()
    for i, dz in enumerate(dz_list):
        out = out + np.asarray(gamma_rows[i], np.float64)[None, None, :] * np.asarray(dz, np.float64)
    return out


def triangular_lazy_np(x0, alpha_list, beta_list, dz_list, g):
    """Workspace inputs z_l of the non-shared lazy schedule (local_thc.py:1495-1510;
    lthc_v2/model.py:256-267): z_l = R_l(x0) + sum_{j<l} gamma[l, j] dz_j, and X_L."""
    gam = gamma_matrix_np(alpha_list, beta_list)
    zs = [triangular_np(read_np(x0, alpha_list[l], g), dz_list[:l], gam[l]) for l in range(len(alpha_list))]
    return zs, final_accumulate_np(x0, dz_list, beta_list)


def interface_bwd_np(x0, alpha, dz_list, beta_list, grad_xl, grad_z_list, g):
    """Closed-form backward of the lazy interface.

    Given G = dL/dX_L and H_l = dL/dZ_l (l < L; Z_L feeds nothing), with the
    suffix sums S_l = sum_{j >= l} H_j:
      dX0      = G + R^T S_0
      d(dZ_l)  = P_l^T G + gamma_l * S_{l+1}
      d(beta_l)= sum G dZ_l + (sum S_{l+1} dZ_l) * alpha
      d(alpha) = sum X0 S_0 + sum_l (sum S_{l+1} dZ_l) * beta_l
    """
    L = len(dz_list)
    h = x0.shape[1]
    S = [None] * (L + 1)
    S[L] = np.zeros_like(np.asarray(grad_z_list[0], np.float64))
    for l in range(L - 1, -1, -1):
        S[l] = S[l + 1] + np.asarray(grad_z_list[l], np.float64)
    dx0 = np.asarray(grad_xl, np.float64) + write_np(S[0], alpha, h)
    dalpha = weight_grad_np(x0, S[0], g)
    ddz, dbeta = [], []
    for l in range(L):
        gam = gamma_np(alpha, beta_list[l])
        ddz.append(read_np(grad_xl, beta_list[l], g) + gam[None, None, :] * S[l + 1])
        dgam = (S[l + 1] * np.asarray(dz_list[l], np.float64)).sum(axis=(0, 1))
        dbeta.append(weight_grad_np(grad_xl, dz_list[l], g) + dgam[:, None] * np.asarray(alpha, np.float64))
        dalpha = dalpha + dgam[:, None] * np.asarray(beta_list[l], np.float64)
    return {"x0": dx0, "alpha": dalpha, "dz": ddz, "beta": dbeta}


# ---------------------------------------------------------------------------
# C restatement (lthc_oracle.c) through ctypes
# ---------------------------------------------------------------------------
def build(verbose: bool = False) -> str:
    """Compile lthc_oracle.c into liblthc_oracle.so next to it."""
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O3", "-fopenmp", "-fPIC", "-shared", "-o", tmp, SRC]
    subprocess.run(cmd, check=True, capture_output=not verbose)
    os.replace(tmp, LIB)
    return LIB


_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} is not built; run oracle.oracle.build()")
        lib = ctypes.CDLL(LIB)
        vp, i64, ci = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        pp = ctypes.POINTER(ctypes.c_void_p)
        lib.oracle_set_threads.argtypes = [ci]
        lib.oracle_max_threads.restype = ci
        lib.oracle_read.argtypes = [vp, vp, vp, i64, i64, i64, i64]
        lib.oracle_write.argtypes = [vp, pp, pp, vp, i64, i64, i64, i64, ci]
        lib.oracle_read_multi.argtypes = [vp, pp, pp, i64, i64, i64, i64, ci]
        lib.oracle_weight_grad.argtypes = [vp, pp, vp, i64, i64, i64, i64, ci]
        lib.oracle_gamma.argtypes = [vp, pp, vp, i64, i64, ci]
        lib.oracle_recur.argtypes = [vp, vp, vp, vp, i64, i64]
        lib.oracle_recur_bwd.argtypes = [vp, vp, vp, vp, vp, i64, i64]
        _LIB = lib
    return _LIB


def set_threads(n: int) -> None:
    _lib().oracle_set_threads(int(n))


def max_threads() -> int:
    return int(_lib().oracle_max_threads())


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def _ptrs(arrs):
    return (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])


def Cread(x, alpha, g: int) -> np.ndarray:
    x, alpha = _f32(x), _f32(alpha)
    b, h, _, c = x.shape
    z = np.empty((b, g * g, c), np.float32)
    _lib().oracle_read(_ptr(x), _ptr(alpha), _ptr(z), b, g, h // g, c)
    return z


def Cwrite(base, dz_list, beta_list, h: int | None = None) -> np.ndarray:
    """out = base + sum_l P_l(dz_l); base may be None (then ``h`` gives the high-res side)."""
    dz_list = [_f32(d) for d in dz_list]
    beta_list = [_f32(bt) for bt in beta_list]
    b, m, c = dz_list[0].shape
    if base is not None:
        base = _f32(base)
        h = base.shape[1]
    g, s = grid_of(h, m)
    out = np.empty((b, h, h, c), np.float32)
    _lib().oracle_write(
        _ptr(base) if base is not None else None, _ptrs(dz_list), _ptrs(beta_list), _ptr(out), b, g, s, c, len(dz_list)
    )
    return out


def Cread_multi(gr, w_list, g: int) -> list[np.ndarray]:
    gr = _f32(gr)
    w_list = [_f32(w) for w in w_list]
    b, h, _, c = gr.shape
    outs = [np.empty((b, g * g, c), np.float32) for _ in w_list]
    _lib().oracle_read_multi(_ptr(gr), _ptrs(w_list), _ptrs(outs), b, g, h // g, c, len(w_list))
    return outs


def Cweight_grad(high, low_list, g: int) -> np.ndarray:
    """[L, C, K] float32."""
    high = _f32(high)
    low_list = [_f32(lo) for lo in low_list]
    b, h, _, c = high.shape
    s = h // g
    gw = np.empty((len(low_list), c, s * s), np.float32)
    _lib().oracle_weight_grad(_ptr(high), _ptrs(low_list), _ptr(gw), b, g, s, c, len(low_list))
    return gw


def Cgamma(alpha, beta_list) -> np.ndarray:
    alpha = _f32(alpha)
    beta_list = [_f32(bt) for bt in beta_list]
    c, k = alpha.shape
    out = np.empty((len(beta_list), c), np.float32)
    _lib().oracle_gamma(_ptr(alpha), _ptrs(beta_list), _ptr(out), c, k, len(beta_list))
    return out


def Crecur(z, dz, gamma) -> np.ndarray:
    z, dz, gamma = _f32(z), _f32(dz), _f32(gamma)
    c = z.shape[-1]
    out = np.empty_like(z)
    _lib().oracle_recur(_ptr(z), _ptr(dz), _ptr(gamma), _ptr(out), z.size // c, c)
    return out


def Crecur_bwd(gr, dz, gamma):
    gr, dz, gamma = _f32(gr), _f32(dz), _f32(gamma)
    c = gr.shape[-1]
    gdz = np.empty_like(gr)
    gg = np.empty((c,), np.float32)
    _lib().oracle_recur_bwd(_ptr(gr), _ptr(dz), _ptr(gamma), _ptr(gdz), _ptr(gg), gr.size // c, c)
    return gdz, gg


# ---------------------------------------------------------------------------
# Seeded inputs of the benchmark configurations (one CPU torch.Generator, fixed
# draw order: X0, alpha, beta stack, dZ stack, then upstream gradients)
# ---------------------------------------------------------------------------
def make_inputs(B: int, G: int, C: int, L: int, seed: int = 0, grads: bool = False, S: int = 4):
    """float32 numpy inputs drawn with torch's CPU generator (bit-identical on every host)."""
    import torch

    gen = torch.Generator().manual_seed(seed)
    H = G * S
    x0 = torch.randn((B, H, H, C), generator=gen)
    alpha = torch.randn((C, S * S), generator=gen) * 0.01 + 1.0 / 16.0
    betas = torch.randn((L, C, S * S), generator=gen) * 0.02
    dzs = torch.randn((L, B, G * G, C), generator=gen) * 0.02
    out = {"x0": x0.numpy(), "alpha": alpha.numpy(), "beta": betas.numpy(), "dz": dzs.numpy()}
    if grads:
        out["grad_xl"] = (torch.randn((B, H, H, C), generator=gen) * 1e-3).numpy()
        out["grad_z"] = (torch.randn((L, B, G * G, C), generator=gen) * 1e-3).numpy()
    return out
