"""Benchmark configurations 3 and 5 at their own sizes, bf16 activations, fp32 weights:
  configuration 3: B=64, 64x64 / 16x16, C=768, L=12;
  configuration 5: B=32, 128x128 / 32x32, C=1024, L=24 (the depth-24 kernels over every grid step).
The interface forward + backward through the model's autograd ops and through the single-pass C entry point
(lthc_interface_bwd), each against the closed-form backward evaluated by the C oracle on the same bf16 inputs.

Closed form (local_thc.py:1211-1223, 1325-1328, 1368-1372 differentiated; G = dL/dX_L, H_l = dL/dZ_l,
S_l = sum_{j >= l} H_j):
    dX0 = G + R^T S_0,   d dZ_l = P_l^T G + gamma_l S_{l+1},
    d beta_l = sum G dZ_l + alpha * sum S_{l+1} dZ_l,   d alpha = sum X0 S_0 + sum_l beta_l * sum S_{l+1} dZ_l.
The C oracle (oracle/lthc_oracle.c, fp64 accumulation) supplies R^T, P_l^T and the cell sums; the suffix sums and
the gamma-term sums run in float64 here.

Bounds, in units of the reference's largest magnitude (the gradients are O(1e-3)): the GPU path rounds the suffix
sums, the recurrence gradients and its outputs to bf16 and the model path uses the bf16 gamma of the autograd
sequence, so activation gradients are held to max |d| <= 1e-2 max|ref| and mean |d| <= 4e-3 mean|ref| (one bf16 unit roundoff), weight
gradients (fp32 sums over 16384 or 32768 cells of bf16 products) to max |d| <= 1e-2 max|ref|.  A dropped term (the
gamma term, the base G in dX0, a layer of the suffix) moves them by O(1).
"""

import ctypes

import numpy as np
import pytest
import torch

from flowmatching_lthc_amd import _abi, ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16 = torch.bfloat16
CONFIGS = {"configuration3": (64, 16, 768, 12, 3), "configuration5": (32, 32, 1024, 24, 5)}  # B, G, C, L, seed


@pytest.fixture(scope="module", params=list(CONFIGS))
def full(request, coracle):
    """The configuration's draws (X0 ~ N(0,1), alpha ~ N(1/16, 0.01), beta_l ~ N(0, 0.02), dZ_l ~ N(0, 0.02), G_L and
    H_l ~ N(0, 1e-3)) from a seeded generator on the device (the host copies are the same bits), and the closed-form
    reference on the host."""
    B, G, C, L, seed = CONFIGS[request.param]
    print(f"case {request.param}: B={B} G={G} C={C} L={L} inputs and closed-form reference", flush=True)
    coracle.set_threads(min(16, coracle.max_threads()))
    gen = torch.Generator(device=DEV).manual_seed(seed)
    rn = lambda *shape: torch.randn(shape, generator=gen, device=DEV)  # noqa: E731
    t = {
        "x0": rn(B, 4 * G, 4 * G, C).to(BF16).cpu(),
        "alpha": (rn(C, 16) * 0.01 + 1.0 / 16.0).cpu(),
        "beta": [(rn(C, 16) * 0.02).cpu() for _ in range(L)],
        "dz": [(rn(B, G * G, C) * 0.02).to(BF16).cpu() for _ in range(L)],
        "gx": (rn(B, 4 * G, 4 * G, C) * 1e-3).to(BF16).cpu(),
        "gz": [(rn(B, G * G, C) * 1e-3).to(BF16).cpu() for _ in range(L)],
    }
    d = {"alpha": t["alpha"].numpy(), "beta": np.stack([b.numpy() for b in t["beta"]])}
    h = lambda x: x.float().numpy()  # noqa: E731  (bf16 values, exactly)
    x0, gx = h(t["x0"]), h(t["gx"])
    dzs, gzs = [h(z) for z in t["dz"]], [h(z) for z in t["gz"]]
    alpha, betas = d["alpha"], list(d["beta"])
    S = [None] * (L + 1)
    acc = np.zeros(gzs[0].shape, np.float64)
    S[L] = acc.astype(np.float32)
    for l in reversed(range(L)):
        acc += gzs[l]
        S[l] = acc.astype(np.float32)
    gam = coracle.Cgamma(alpha, betas).astype(np.float64)
    ref = {"x0": coracle.Cwrite(gx, [S[0]], [alpha])}
    pt = coracle.Cread_multi(gx, betas, G)
    dgam = [(S[l + 1].astype(np.float64) * dzs[l]).sum(axis=(0, 1)) for l in range(L)]
    ref["dz"] = [pt[l] + gam[l][None, None, :] * S[l + 1] for l in range(L)]
    gw = coracle.Cweight_grad(gx, dzs, G)
    ref["beta"] = [gw[l] + dgam[l][:, None] * alpha for l in range(L)]
    ref["alpha"] = coracle.Cweight_grad(x0, [S[0]], G)[0] + sum(dgam[l][:, None] * betas[l] for l in range(L))
    return (B, G, C, L), t, ref


def _check(name, got, ref, act):
    got = got.float().cpu().numpy() if isinstance(got, torch.Tensor) else got
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    scale = np.abs(ref).max()
    assert d.max() <= 1e-2 * scale, f"{name}: max err {d.max() / scale:.3e} of max|ref|"
    if act:
        assert d.mean() <= 4e-3 * np.abs(ref).mean(), f"{name}: mean err {d.mean() / np.abs(ref).mean():.3e}"


@pytest.mark.timeout(600)
def test_autograd_backward_full_size(full):
    """The model's lazy-forward ops (read_with_residual, the one-launch bf16 gamma, the split recurrence steps, the
    12-pointer materialisation at depth 12 and the list op otherwise) and torch.autograd.grad over
    (X_L, Z_0..Z_{L-1}), as bench.py's training leg runs."""
    (B, G, C, L), t, ref = full
    x0 = t["x0"].to(DEV).requires_grad_()
    alpha = t["alpha"].to(DEV).requires_grad_()
    betas = [b.to(DEV).requires_grad_() for b in t["beta"]]
    dzs = [z.to(DEV).requires_grad_() for z in t["dz"]]
    x0v, z = ops.read_with_residual(x0, alpha.to(BF16))
    gam = ops.lazy_gamma_rounded(alpha, betas, BF16).unbind(0)
    zs, dzv = [z], []
    for l in range(L):
        z, zb, dv = ops.lazy_workspace_step(z, dzs[l], gam[l], split=True)
        zs.append(zb)
        dzv.append(dv)
    xl = ops.final_accumulate_b4_12_traceable(x0v, *dzv, *betas) if L == 12 else ops.final_accumulate_list(x0v, dzv, betas)
    grads = torch.autograd.grad([xl] + zs[:L], [x0, alpha] + betas + dzs, [t["gx"].to(DEV)] + [g.to(DEV) for g in t["gz"]])
    torch.cuda.synchronize()
    _check("dX0", grads[0], ref["x0"], True)
    _check("dalpha", grads[1], ref["alpha"], False)
    for l in range(L):
        _check(f"dbeta_{l}", grads[2 + l], ref["beta"][l], False)
        _check(f"d dZ_{l}", grads[2 + L + l], ref["dz"][l], True)


@pytest.mark.timeout(300)
def test_single_pass_backward_full_size(full):
    """lthc_interface_bwd (the single-pass tile kernel, then dalpha and the gamma terms) at the configuration's size."""
    (B, G, C, L), t, ref = full
    lib = _abi.load()
    x0, gx = t["x0"].to(DEV), t["gx"].to(DEV)
    dzs, gzs = [z.to(DEV) for z in t["dz"]], [g.to(DEV) for g in t["gz"]]
    alpha, betas = t["alpha"].to(DEV), [b.to(DEV) for b in t["beta"]]
    dx0 = torch.empty_like(x0)
    ddz = [torch.empty_like(z) for z in dzs]
    da = torch.empty((C, 16), device=DEV)
    db = torch.empty((L, C, 16), device=DEV)
    ws = torch.empty((int(lib.lthc_interface_workspace_bytes(B, G, 4, C, L)),), device=DEV, dtype=torch.uint8)
    gz = (ctypes.c_void_p * L)(*[g.data_ptr() for g in gzs])
    rc = lib.lthc_interface_bwd(
        gx.data_ptr(), gz, _abi.code(gx), x0.data_ptr(), _abi.ptr_array(dzs), alpha.data_ptr(), _abi.ptr_array(betas),
        _abi.code(alpha), dx0.data_ptr(), _abi.ptr_array(ddz), da.data_ptr(), db.data_ptr(), B, G, 4, C, L,
        ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream,
    )  # fmt: skip
    _abi.check(rc, "lthc_interface_bwd")
    torch.cuda.synchronize()
    _check("dX0", dx0, ref["x0"], True)
    _check("dalpha", da, ref["alpha"], False)
    for l in range(L):
        _check(f"dbeta_{l}", db[l], ref["beta"][l], False)
        _check(f"d dZ_{l}", ddz[l], ref["dz"][l], True)
