"""Every depth the C ABI takes, through the per-op and whole-interface entry points, against the oracle (MI355X only).

The materialisation and its backward pick a kernel by depth bucket: the whole-cell kernel with its weights in
VGPRs for depths 1, 2, 4, 8 and 12 (exact and padded buckets), two tap groups for depths 13-16, the deep kernel
with part of its weights in LDS for depths 17-24 with a base, and the block-range kernels above depth 24.  The
backward's tile kernel has 4 wavefronts up to depth 12 and 8 above (with gbeta's layers in two 16-wide blocks of
matrix-core columns above depth 16).  This sweep runs each depth from 1 to 25, plus
33 and 48 (the largest the ABI takes), on one sample of the B/4 geometry (G = 16) at C = 256, with bf16 activations
and fp32 weights (the released autocast run), fp16 activations and weights, and fp32 throughout, and checks:
- lthc_materialise_fwd with and without a base against X0 + sum_l P_l dZ_l (local_thc.py:1368-1372;
  local_thc_triton_kernels.py:317-405), the oracle evaluated in float64 on the rounded inputs;
- lthc_materialise_bwd's gdZ_l = sum_k beta_l G and gbeta_l = sum_cells G dZ_l
  (local_thc_triton_kernels.py:512-680);
- lthc_read_multi_fwd and lthc_weight_grad, the same two quantities from the per-op kernels.
Tolerances as in test_gpu_parity: 16-bit outputs within one rounding of the fp64 value (and 2e-2 absolute), fp32
outputs and weight gradients within 1e-5 of max|ref|.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O

from . import capi
from .test_gpu_parity import BF16, F32, assert_bf16, assert_f32, dev, host, rounded

pytestmark = pytest.mark.gpu

DEPTHS = list(range(1, 26)) + [33, 48]


F16 = torch.float16


def assert_act(got, ref, xdt, what):
    """16-bit outputs within one rounding of the fp64 value (|d| <= u|ref| + 1e-5, u = 2^-8 for bf16 and 2^-11 for
    fp16, and 2e-2 absolute); fp32 outputs within 1e-5 of max|ref|."""
    if xdt == F32:
        assert_f32(got, ref, what=what)
        return
    if xdt == BF16:
        assert_bf16(got, ref, what=what)
        return
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    assert d.max() <= 2e-2, f"{what}: max abs err {d.max():.3e} > 2e-2"
    bad = int((d > 2.0**-11 * np.abs(ref) + 1e-5).sum())
    assert bad == 0, f"{what}: {bad} elements exceed 2^-11|ref| + 1e-5"


@pytest.mark.parametrize("xdt,wdt", [(BF16, F32), (F16, F16), (F32, F32)], ids=["bf16-f32w", "f16-f16w", "f32"])
@pytest.mark.parametrize("L", DEPTHS)
def test_every_depth_materialise_and_backward(L, xdt, wdt):
    B, G, C = 1, 16, 256
    print(f"case depth L={L} B={B} G={G} C={C} activations {xdt}, weights {wdt}", flush=True)
    d = O.make_inputs(B, G, C, L, seed=100 + L, grads=True)
    x0h = rounded(d["x0"], xdt)
    dzh = [rounded(d["dz"][l], xdt) for l in range(L)]
    gh = rounded(d["grad_xl"], xdt)
    betas_np = [rounded(d["beta"][l], wdt) for l in range(L)]

    x0 = dev(x0h, xdt)
    dzs = [dev(z, xdt) for z in dzh]
    gr = dev(gh, xdt)
    betas = [dev(b, wdt) for b in betas_np]

    ref = O.final_accumulate_np(x0h, dzh, betas_np)
    assert_act(host(capi.materialise(x0, dzs, betas)), ref, xdt, what=f"materialise L={L}")
    if L <= 24:  # a NULL base takes up to 24 layers (the adjoint of the multi-weight read)
        ref0 = O.final_accumulate_np(np.zeros_like(x0h), dzh, betas_np)
        assert_act(host(capi.materialise(None, dzs, betas)), ref0, xdt, what=f"materialise without base L={L}")

    gdz, gb = capi.materialise_bwd(gr, dzs, betas)
    multi = capi.read_multi(gr, betas)
    wg = capi.weight_grad(gr, dzs)
    for l in range(L):
        ref_gdz = O.read_np(gh, betas_np[l], G)
        assert_act(host(gdz[l]), ref_gdz, xdt, what=f"materialise_bwd gdZ_{l} L={L}")
        assert_act(host(multi[l]), ref_gdz, xdt, what=f"read_multi gdZ_{l} L={L}")
        ref_gb = O.weight_grad_np(gh, dzh[l], G)
        assert_f32(host(gb[l]), ref_gb, what=f"materialise_bwd gbeta_{l} L={L}")
        assert_f32(host(wg[l]), ref_gb, what=f"weight_grad gbeta_{l} L={L}")
    # the two backward paths share their FMA order for gdZ: bitwise equal
    for l in range(L):
        assert torch.equal(gdz[l], multi[l]), f"materialise_bwd and read_multi gdZ_{l} differ at L={L}"


def assert_grad(got, ref, what, weight=False):
    """Bounds of tests/test_gpu_full_size.py: the bf16 path rounds the suffix sums and its outputs, so activation
    gradients are held to max|d| <= 1e-2 max|ref| and mean|d| <= 4e-3 mean|ref|, fp32 weight gradients to
    max|d| <= 1e-2 max|ref|; a dropped term moves them by O(1)."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    assert d.max() <= 1e-2 * np.abs(ref).max(), f"{what}: max|d| {d.max():.3e} vs max|ref| {np.abs(ref).max():.3e}"
    if not weight:
        assert d.mean() <= 4e-3 * np.abs(ref).mean(), f"{what}: mean|d| {d.mean():.3e} vs mean|ref| {np.abs(ref).mean():.3e}"


@pytest.mark.parametrize("L", list(range(1, 26)) + [33])
def test_every_depth_whole_interface(L):
    """lthc_interface_fwd (one pass at depths <= 12 and 24, composed at the padded depths 13-23 and above 24) and
    lthc_interface_bwd (the single-pass tile kernel up to depth 24, the composed chain above) at every depth:
    Z_0 = R(X0), each step Z_{l+1} = Z_l + gamma_l dZ_l from the returned bf16 Z_l (local_thc.py:1211-1223,
    1325-1328), X_L (:1368-1372), and the closed-form backward (oracle.interface_bwd_np) on the same bf16 inputs."""
    B, G, C = 1, 16, 256
    print(f"case whole interface L={L} B={B} G={G} C={C} bf16 activations, fp32 weights", flush=True)
    d = O.make_inputs(B, G, C, L, seed=200 + L, grads=True)
    x0h = rounded(d["x0"], BF16)
    dzh = [rounded(d["dz"][l], BF16) for l in range(L)]
    gxh = rounded(d["grad_xl"], BF16)
    gzh = [rounded(d["grad_z"][l], BF16) for l in range(L)]
    alpha_np, betas_np = d["alpha"], [d["beta"][l] for l in range(L)]
    x0, gx = dev(x0h, BF16), dev(gxh, BF16)
    dzs, gzs = [dev(z, BF16) for z in dzh], [dev(z, BF16) for z in gzh]
    alpha, betas = dev(alpha_np, F32), [dev(b, F32) for b in betas_np]

    zs, xl = capi.interface_fwd(x0, alpha, betas, dzs)
    assert_bf16(host(zs[0]), O.read_np(x0h, alpha_np, G), what=f"Z_0 L={L}")
    for l in range(L):
        ref = O.lazy_update_np(host(zs[l]), dzh[l], O.gamma_np(alpha_np, betas_np[l]))
        assert_bf16(host(zs[l + 1]), ref, what=f"Z_{l + 1} L={L}")
    assert_bf16(host(xl), O.final_accumulate_np(x0h, dzh, betas_np), what=f"X_L L={L}")

    dx0, ddz, da, db = capi.interface_bwd(gx, gzs, x0, dzs, alpha, betas)
    ref = O.interface_bwd_np(x0h, alpha_np, dzh, betas_np, gxh, gzh, G)
    assert_grad(host(dx0), ref["x0"], f"dX0 L={L}")
    assert_grad(host(da), ref["alpha"], f"dalpha L={L}", weight=True)
    for l in range(L):
        assert_grad(host(ddz[l]), ref["dz"][l], f"d dZ_{l} L={L}")
        assert_grad(host(db[l]), ref["beta"][l], f"dbeta_{l} L={L}", weight=True)
