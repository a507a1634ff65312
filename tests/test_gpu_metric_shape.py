"""The whole-interface C entry points at the metric shape: B=256, 64x64 / 16x16, C=768, L=12, bf16 activations,
fp32 weights (the shape bench.py times).  Its hi-res tensors (1.61 GB) put the kernels' 32-bit byte offsets near their
largest values, which the smaller configurations never reach.

- lthc_interface_fwd (the one-pass iface_fwd_kernel) equals the per-op chain it replaces bit for bit (lthc_read_fwd,
  lthc_gamma, twelve lthc_recur_fwd, lthc_materialise_fwd), and its X_L and Z_0 lie within one bf16 rounding of the C
  oracle on the first, a middle and the last sample.
- lthc_interface_bwd (the single-pass bwd_tile_kernel, then dalpha and the gamma terms) matches the closed form of
  the interface backward (local_thc.py:1211-1223, 1325-1328, 1368-1372 differentiated; see test_gpu_full_size.py):
  the activation gradients on the same three samples, the weight gradients summed over the whole batch.  The bounds
  are the full-size tests': max |d| <= 1e-2 max|ref| (and mean |d| <= 4e-3 mean|ref| for activations).
- the non-shared forward's triangular sums (ws_acc_fwd_flat_kernel, fp32 gamma) at the widest and narrowest width:
  within one bf16 rounding of an fp64 sum, and exact where gamma is zero.
"""

import numpy as np
import pytest
import torch

from tests import capi

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16 = torch.bfloat16
B, G, C, L = 256, 16, 768, 12
SAMPLES = (0, 131, 255)


def _bf16_bound(got: np.ndarray, ref: np.ndarray, what: str):
    """One RNE rounding to bf16 after an fp32 sum: |d| <= 2^-8 |ref| + 1e-5, and the stated 2e-2 absolute bar."""
    d = np.abs(got - ref)
    assert d.max() <= 2e-2, f"{what}: max abs err {d.max():.3e}"
    bad = d > 2.0**-8 * np.abs(ref) + 1e-5
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond one bf16 rounding"


def _check(name, got, ref, act):
    got = got.float().cpu().numpy() if isinstance(got, torch.Tensor) else got
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    scale = np.abs(ref).max()
    assert d.max() <= 1e-2 * scale, f"{name}: max err {d.max() / scale:.3e} of max|ref|"
    if act:
        assert d.mean() <= 4e-3 * np.abs(ref).mean(), f"{name}: mean err {d.mean() / np.abs(ref).mean():.3e}"


@pytest.fixture(scope="module")
def inputs():
    print(f"metric shape B={B} G={G} C={C} L={L}: drawing inputs", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(256)
    rn = lambda *shape: torch.randn(shape, generator=gen, device=DEV)  # noqa: E731
    x0 = rn(B, 4 * G, 4 * G, C).to(BF16)
    alpha = rn(C, 16) * 0.01 + 1.0 / 16.0
    betas = [rn(C, 16) * 0.02 for _ in range(L)]
    dzs = [(rn(B, G * G, C) * 0.02).to(BF16) for _ in range(L)]
    return x0, alpha, betas, dzs, gen


@pytest.mark.timeout(600)
def test_interface_fwd_metric_shape(inputs, coracle):
    x0, alpha, betas, dzs, _ = inputs
    zs, xl = capi.interface_fwd(x0, alpha, betas, dzs)
    z = capi.read(x0, alpha)
    gam = capi.gamma(alpha, betas)
    assert torch.equal(zs[0], z), "Z_0 differs from lthc_read_fwd"
    for l in range(L):
        z = capi.recur(z, dzs[l], gam[l])
        assert torch.equal(zs[l + 1], z), f"Z_{l + 1} differs from the recurrence steps"
    del z
    assert torch.equal(xl, capi.materialise(x0, dzs, betas)), "X_L differs from lthc_materialise_fwd"
    print("one-pass forward equals the per-op chain; oracle samples", flush=True)
    coracle.set_threads(min(16, coracle.max_threads()))
    a, bs = alpha.cpu().numpy(), [b.cpu().numpy() for b in betas]
    for b in SAMPLES:
        x0h = x0[b : b + 1].float().cpu().numpy()
        dzh = [d[b : b + 1].float().cpu().numpy() for d in dzs]
        _bf16_bound(xl[b : b + 1].float().cpu().numpy(), coracle.Cwrite(x0h, dzh, bs), f"X_L[{b}]")
        _bf16_bound(zs[0][b : b + 1].float().cpu().numpy(), coracle.Cread(x0h, a, G), f"Z_0[{b}]")


@pytest.mark.timeout(600)
def test_interface_bwd_metric_shape(inputs, coracle):
    x0, alpha, betas, dzs, gen = inputs
    rn = lambda *shape: torch.randn(shape, generator=gen, device=DEV)  # noqa: E731
    gx = (rn(B, 4 * G, 4 * G, C) * 1e-3).to(BF16)
    gzs = [(rn(B, G * G, C) * 1e-3).to(BF16) for _ in range(L)]
    dx0, ddz, da, db = capi.interface_bwd(gx, gzs, x0, dzs, alpha, betas)
    torch.cuda.synchronize()
    print("single-pass backward done; closed form on the host", flush=True)
    coracle.set_threads(min(16, coracle.max_threads()))
    a, bs = alpha.cpu().numpy(), [b.cpu().numpy() for b in betas]
    gam = coracle.Cgamma(a, bs).astype(np.float64)
    # suffix sums S_l = sum_{j >= l} H_j (float64, rounded to fp32 as the oracle's inputs), over the whole batch
    acc = np.zeros((B, G * G, C), np.float64)
    S = [None] * (L + 1)
    S[L] = acc.astype(np.float32)
    for l in reversed(range(L)):
        acc += gzs[l].float().cpu().numpy()
        S[l] = acc.astype(np.float32)
    del acc
    dzh = [d.float().cpu().numpy() for d in dzs]
    dgam = [(S[l + 1].astype(np.float64) * dzh[l]).sum(axis=(0, 1)) for l in range(L)]
    gxh = gx.float().cpu().numpy()
    gw = coracle.Cweight_grad(gxh, dzh, G)
    for l in range(L):
        _check(f"dbeta_{l}", db[l], gw[l] + dgam[l][:, None] * a, False)
    del gw
    x0h = x0.float().cpu().numpy()
    ref_da = coracle.Cweight_grad(x0h, [S[0]], G)[0] + sum(dgam[l][:, None] * bs[l] for l in range(L))
    _check("dalpha", da, ref_da, False)
    del x0h
    print("weight gradients match; activation samples", flush=True)
    for b in SAMPLES:
        g1 = gxh[b : b + 1]
        _check(f"dX0[{b}]", dx0[b : b + 1], coracle.Cwrite(g1, [S[0][b : b + 1]], [a]), True)
        pt = coracle.Cread_multi(g1, bs, G)
        for l in range(L):
            _check(f"d dZ_{l}[{b}]", ddz[l][b : b + 1], pt[l] + gam[l][None, None, :] * S[l + 1][b : b + 1], True)


@pytest.mark.parametrize("active", [11, 1])
def test_triangular_sums_metric_shape(active):
    """The non-shared forward's triangular sum at the metric shape with fp32 gamma (the model's case under autocast:
    the two-rows-per-thread kernel), against an fp64 sum on the GPU: within one bf16 rounding everywhere (the
    kernel's fp32 fma chain is exact to well below it), and a zero gamma row returns the base bit for bit."""
    from flowmatching_lthc_amd import ops_triangular as T

    print(f"case triangular sum metric shape B={B} active={active}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(100 + active)
    base = torch.randn((B, G * G, C), generator=gen, device=DEV).to(BF16)
    dzs = [(torch.randn((B, G * G, C), generator=gen, device=DEV) * 0.02).to(BF16) for _ in range(active)]
    gamma = torch.randn((12, C), generator=gen, device=DEV) * 0.1 + 1.0
    gamma[:, 5] = 0.0  # channel 5: every term zero
    slots = tuple(dzs[j] if j < active else torch.zeros_like(base) for j in range(12))
    out = T.triangular_accumulate_b4_12_ptr_active_traceable_ops[active - 1](base, *slots, gamma)
    assert out.dtype == BF16
    assert torch.equal(out[..., 5], base[..., 5])
    for b0 in range(0, B, 64):  # the fp64 reference in 64-sample slices
        ref = base[b0 : b0 + 64].double()
        for j in range(active):
            ref += gamma[j].double() * dzs[j][b0 : b0 + 64].double()
        got = out[b0 : b0 + 64].double()
        d = (got - ref).abs()
        assert d.max().item() <= 2e-2
        assert bool((d <= 2.0**-8 * ref.abs() + 1e-5).all()), f"slice {b0}: beyond one bf16 rounding"
