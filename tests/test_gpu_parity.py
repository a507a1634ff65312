"""GPU parity of the HIP kernels against the CPU oracle (MI355X only).

Tolerances (north star): fp32 results must satisfy max|got - ref| / max|ref|
<= 1e-5 per tensor (an elementwise relative bound is ill-conditioned where the
reference crosses zero); bf16 results must satisfy max|got - ref| <= 2e-2
against the oracle evaluated in fp64 on the same bf16-rounded inputs, and the
tighter elementwise bound |got - ref| <= 2^-8 |ref| + 1e-5 (one
round-to-nearest-even to bf16 after fp32 accumulation).
Inputs come from oracle.make_inputs (seeded CPU torch.Generator), so the CPU
and the GPU see identical bits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from flowmatching_lthc_amd import _abi, ops
from oracle import oracle as O

from . import capi

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
F32, BF16 = torch.float32, torch.bfloat16


def dev(a, dtype=F32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV).to(dtype)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def rounded(a, dtype):
    """The values the GPU sees after casting to `dtype`, as fp32 numpy."""
    return host(dev(a, dtype))


def assert_f32(got, ref, tol=1e-5, what=""):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), 1e-30)
    err = np.abs(got - ref).max() / scale
    assert err <= tol, f"{what}: max|d|/max|ref| = {err:.3e} > {tol}"


def assert_bf16(got, ref, what=""):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    assert d.max() <= 2e-2, f"{what}: max abs err {d.max():.3e} > 2e-2"
    bound = 2.0**-8 * np.abs(ref) + 1e-5
    bad = int((d > bound).sum())
    assert bad == 0, f"{what}: {bad} elements exceed 2^-8|ref| + 1e-5 (worst {np.max(d - bound):.3e})"


@pytest.fixture(scope="module", autouse=True)
def _oracle_built(coracle):
    coracle.set_threads(16)
    yield


def cfg(B, G, C, L, seed=0, grads=False):
    return O.make_inputs(B, G, C, L, seed=seed, grads=grads)


# ---------------------------------------------------------------------------
# configuration 1: read + one write, fp32, B=2
# ---------------------------------------------------------------------------
def test_config1_read_and_write_fp32(coracle):
    d = cfg(2, 16, 768, 1)
    x0, alpha, beta, dz = d["x0"], d["alpha"], d["beta"][0], d["dz"][0]
    z = capi.read(dev(x0), dev(alpha))
    assert_f32(host(z), coracle.Cread(x0, alpha, 16), what="read")
    xl = capi.materialise(dev(x0), [dev(dz)], [dev(beta)])
    assert_f32(host(xl), coracle.Cwrite(x0, [dz], [beta]), what="write_add")
    w = capi.materialise(None, [dev(dz)], [dev(beta)])
    assert_f32(host(w), coracle.Cwrite(None, [dz], [beta], h=64), what="write")


# ---------------------------------------------------------------------------
# configuration 2: full lazy interface forward, bf16, B=32, L=12
# ---------------------------------------------------------------------------
def test_config2_lazy_interface_bf16(coracle):
    B, G, C, L = 32, 16, 768, 12
    d = cfg(B, G, C, L)
    x0 = dev(d["x0"], BF16)
    alpha = dev(d["alpha"])  # fp32 weights, as the released model passes them
    betas = [dev(b) for b in d["beta"]]
    dzs = [dev(z, BF16) for z in d["dz"]]
    x0h, dzh = host(x0), [host(z) for z in dzs]

    z = capi.read(x0, alpha)
    assert_bf16(host(z), coracle.Cread(x0h, d["alpha"], G), what="read")

    gam = capi.gamma(alpha, betas)
    assert_f32(host(gam), coracle.Cgamma(d["alpha"], list(d["beta"])), tol=1e-6, what="gamma")

    for l in range(L):  # each step against the oracle fed the same bf16 Z_l
        zn = capi.recur(z, dzs[l], gam[l])
        assert_bf16(host(zn), coracle.Crecur(host(z), dzh[l], host(gam[l])), what=f"recurrence step {l}")
        z = zn

    xl = capi.materialise(x0, dzs, betas)
    assert_bf16(host(xl), coracle.Cwrite(x0h, dzh, list(d["beta"])), what="materialise")
    xl_op = ops.final_accumulate_b4_12_traceable(x0, *dzs, *betas)
    assert torch.equal(xl_op, xl)


# ---------------------------------------------------------------------------
# configuration 3: forward + backward at training shape, bf16, B=64, L=12
# ---------------------------------------------------------------------------
def test_config3_materialise_backward_bf16(coracle):
    B, G, C, L = 64, 16, 768, 12
    d = cfg(B, G, C, L, grads=True)
    gout = dev(d["grad_xl"], BF16)
    dzs = [dev(z, BF16) for z in d["dz"]]
    betas = [dev(b) for b in d["beta"]]
    gh, dzh = host(gout), [host(z) for z in dzs]

    gdz = ops.final_accumulate_b4_12_grad_dz_ptr_traceable(gout, *betas)
    ref = coracle.Cread_multi(gh, list(d["beta"]), G)
    for l in range(L):
        assert_bf16(host(gdz[l]), ref[l], what=f"gdZ_{l}")

    gb = ops.final_accumulate_b4_12_grad_beta_ptr_traceable(gout, *dzs)
    gb_ref = coracle.Cweight_grad(gh, dzh, G)
    assert gb.dtype == torch.float32
    assert_f32(host(gb), gb_ref, tol=1e-5, what="gbeta")
    gb2 = ops.final_accumulate_b4_12_grad_beta_ptr_traceable(gout, *dzs)
    assert torch.equal(gb, gb2), "weight-gradient reduction is not deterministic"


def test_config3_read_backward_bf16(coracle):
    B, G, C = 64, 16, 768
    d = cfg(B, G, C, 1, grads=True)
    x0 = dev(d["x0"], BF16)
    gz = dev(d["grad_z"][0], BF16)
    alpha = dev(d["alpha"])
    dx = capi.materialise(None, [gz], [alpha])
    assert_bf16(host(dx), coracle.Cwrite(None, [host(gz)], [d["alpha"]], h=64), what="dX = R^T gZ")
    da = capi.weight_grad(x0, [gz])[0]
    assert_f32(host(da), coracle.Cweight_grad(host(x0), [host(gz)], G)[0], tol=1e-5, what="dalpha")


@pytest.mark.parametrize("fused_open", [False, True, "split"])
def test_interface_autograd_matches_closed_form_fp32(coracle, fused_open):
    """Read op -> 4 recurrence ops -> stacked materialise op, backward through torch autograd.

    fused_open: the model's forward_lazy form -- the read and the materialisation's use of X0 go through
    ops.read_with_residual (dX0 = G_L + R^T gZ0 in one local_read_add pass) and every recurrence step
    through ops.lazy_workspace_step (dZ_l's two gradients summed inside the recurrence backward);
    "split" also takes Z_l for the upstream gradient from the step's branch output (Z_l's two gradients
    summed inside the recurrence backward)."""
    B, G, C, L = 2, 16, 64, 4
    d = cfg(B, G, C, L, seed=3, grads=True)
    t = lambda a: dev(a).requires_grad_(True)  # noqa: E731
    x0_leaf, alpha = t(d["x0"]), t(d["alpha"])
    betas, dzs = t(d["beta"]), [t(z) for z in d["dz"]]
    if fused_open:
        x0, z = ops.read_with_residual(x0_leaf, alpha)
    else:
        x0, z = x0_leaf, ops.local_write_traceable(x0_leaf, alpha)
    zs, dzm = [z], []
    for l in range(L):
        gam = (alpha * betas[l]).sum(-1)
        if fused_open == "split":
            z, zb, dz_m = ops.lazy_workspace_step(z, dzs[l], gam, split=True)
        elif fused_open:
            z, dz_m = ops.lazy_workspace_step(z, dzs[l], gam)
            zb = z
        else:
            z, dz_m = ops.lazy_workspace_update(z, dzs[l], gam), dzs[l]
            zb = z
        zs.append(zb)
        dzm.append(dz_m)
    xl = ops.final_accumulate_b4_traceable(x0, torch.stack(dzm), betas)
    loss = (xl * dev(d["grad_xl"])).sum() + sum((zs[l] * dev(d["grad_z"][l])).sum() for l in range(L))
    loss.backward()
    ref = O.interface_bwd_np(d["x0"], d["alpha"], list(d["dz"]), list(d["beta"]), d["grad_xl"], list(d["grad_z"]), G)
    assert_f32(host(x0_leaf.grad), ref["x0"], what="dX0")
    assert_f32(host(alpha.grad), ref["alpha"], what="dalpha")
    for l in range(L):
        assert_f32(host(dzs[l].grad), ref["dz"][l], what=f"d dZ_{l}")
        assert_f32(host(betas.grad[l]), ref["beta"][l], what=f"dbeta_{l}")


def test_read_add_op_and_backward_bf16(coracle):
    """jit_thc::local_read_add_traceable: x + R^T z in one pass, and its autograd (grad_x = grad_out)."""
    B, G, C = 4, 16, 768
    d = cfg(B, G, C, 1, seed=5, grads=True)
    x, z = dev(d["x0"], BF16), dev(d["dz"][0], BF16)
    w = dev(d["beta"][0]).requires_grad_(True)
    zr, xr = z.clone().requires_grad_(True), x.clone().requires_grad_(True)
    out = ops.local_read_add_traceable(zr, w, xr)
    assert_bf16(host(out), coracle.Cwrite(host(x), [host(z)], [d["beta"][0]]), what="x + R^T z")
    g = dev(d["grad_xl"], BF16)
    out.backward(g)
    assert torch.equal(xr.grad, g)
    assert_bf16(host(zr.grad), coracle.Cread(host(g), d["beta"][0], G), what="grad z = R g")
    assert_f32(host(w.grad), coracle.Cweight_grad(host(g), [host(z)], G)[0], tol=1e-5, what="grad w")


@pytest.mark.parametrize("xdt", [F32, BF16, torch.float16])
@pytest.mark.parametrize("same_gamma_dtype", [False, True])
@pytest.mark.parametrize("C", [768, 260, 12])
def test_recurrence_forward_both_forms(coracle, xdt, same_gamma_dtype, C):
    """z + gamma * dz against the oracle.  16-byte aligned tensors with C a multiple of one 16-byte run take
    the one-shot kernel; 16-bit views shifted by 4 elements (8-byte aligned) and 16-bit C = 260 or 12 take the
    grid-stride kernel.  The two forms agree bit for bit."""
    d = cfg(2, 16, C, 1, grads=True)
    z, dz = dev(d["grad_z"][0] * 50.0, xdt), dev(d["dz"][0], xdt)
    gam = dev(d["alpha"][:, 0] * 3.0)
    if same_gamma_dtype:
        gam = gam.to(xdt)
    ref = coracle.Crecur(host(z), host(dz), host(gam))
    out = capi.recur(z, dz, gam)
    if xdt == F32:
        assert_f32(host(out), ref, what="recurrence fp32")
    else:
        got, r = host(out).astype(np.float64), ref.astype(np.float64)
        bound = 2.0**-8 * np.abs(r) + 1e-5 if xdt == BF16 else 2.0**-11 * np.abs(r) + 1e-7
        assert (np.abs(got - r) <= bound).all(), "recurrence: more than one rounding from the exact result"
        n = z.numel()
        shifted = []
        for t in (z, dz):
            buf = torch.empty(n + 4, device=DEV, dtype=xdt)
            buf[4:].copy_(t.reshape(-1))
            shifted.append(buf[4:].view_as(t))
        out_buf = torch.empty(n + 4, device=DEV, dtype=xdt)
        alt = capi.recur_into(shifted[0], shifted[1], gam, out_buf[4:].view_as(z))
        assert torch.equal(alt, out), "one-shot and grid-stride recurrence differ"


def test_recurrence_backward(coracle):
    d = cfg(8, 16, 768, 2, grads=True)
    g, dz = dev(d["grad_z"][0], BF16), dev(d["dz"][0], BF16)
    gam = dev(d["alpha"][:, 0] * 3.0)
    gdz, gg = capi.recur_bwd(g, dz, gam)
    rgdz, rgg = coracle.Crecur_bwd(host(g), host(dz), host(gam))
    assert_bf16(host(gdz), rgdz, what="gamma * g")
    assert_f32(host(gg), rgg, tol=1e-5, what="ggamma")
    # with the accumulate input: gamma * g + add, one rounding
    add = dev(d["grad_z"][1], BF16)
    gdz2, gg2 = capi.recur_bwd(g, dz, gam, add)
    assert_bf16(host(gdz2), rgdz.astype(np.float64) + host(add), what="gamma * g + add")
    assert torch.equal(gg2, gg)


@pytest.mark.parametrize("xdt", [F32, BF16, torch.float16])
@pytest.mark.parametrize("with_add", [False, True])
@pytest.mark.parametrize("rows_c", [(8 * 256, 768), (3, 12), (1000, 260)])
def test_recurrence_backward_with_branch_gradient(coracle, xdt, with_add, rows_c):
    """lthc_recur_bwd_sum: g + g_branch rounded as autograd's add, then the recurrence backward of that sum --
    bitwise equal to the add followed by lthc_recur_bwd, and the sum's backward against the oracle."""
    rows, c = rows_c
    gen = torch.Generator().manual_seed(rows + c)
    mk = lambda s: dev(torch.randn((rows, c), generator=gen) * s, xdt)  # noqa: E731
    g, gb, dz, add = mk(1e-3), mk(1e-3), mk(0.02), (mk(1e-3) if with_add else None)
    gam = dev(torch.randn((c,), generator=gen) * 0.05)
    gsum, gdz, gg = capi.recur_bwd_sum(g, gb, dz, gam, add)
    assert torch.equal(gsum, g + gb), "g_sum differs from autograd's add"
    gdz_ref, gg_ref = capi.recur_bwd(g + gb, dz, gam, add)
    assert torch.equal(gdz, gdz_ref) and torch.equal(gg, gg_ref), "summed form differs from add + recurrence backward"
    rgdz, rgg = coracle.Crecur_bwd(host(g + gb), host(dz), host(gam))
    if add is not None:
        rgdz = rgdz.astype(np.float64) + host(add)
    if xdt == F32:
        assert_f32(host(gdz), rgdz, what="gamma * (g + g_branch)")
    else:
        assert np.abs(host(gdz) - rgdz).max() <= 2e-2 * max(1.0, np.abs(rgdz).max())
    assert_f32(host(gg), rgg, tol=1e-5, what="ggamma")
    if xdt != F32:  # ggamma written in a 16-bit gamma dtype: the fp32 sum rounded once, as a cast of it
        _, _, gg16 = capi.recur_bwd_sum(g, gb, dz, gam.to(xdt), add, gg_dtype=xdt)
        _, _, gg32 = capi.recur_bwd_sum(g, gb, dz, gam.to(xdt), add)
        assert torch.equal(gg16, gg32.to(xdt))


def test_split_steps_gradients_equal_unsplit_bf16():
    """ops.lazy_workspace_step(split=True): the branch reads the step's second output and the backward sums
    z_next's two gradients inside the recurrence backward.  Every gradient is bitwise that of the unsplit form,
    where autograd adds them (bf16, 6 steps, the last step's z_next unused as in forward_lazy)."""
    B, G, C, L = 4, 16, 768, 6
    gen = torch.Generator().manual_seed(11)
    r = lambda *s, sc=1.0: (torch.randn(s, generator=gen) * sc)  # noqa: E731
    z0 = dev(r(B, G * G, C), BF16)
    dzs = [dev(r(B, G * G, C, sc=0.02), BF16) for _ in range(L)]
    gam = dev(r(L, C, sc=0.05))
    H = [dev(r(B, G * G, C, sc=1e-3), BF16) for _ in range(L)]
    gm = dev(r(B, G * G, C, sc=1e-3), BF16)

    def grads(split):
        leaves = [t.clone().requires_grad_(True) for t in [z0, gam] + dzs]
        z, gm_ = leaves[0], leaves[1]
        zb, zs, dl = z, [], []
        for l in range(L):
            zs.append(zb)
            if split:
                z, zb, d = ops.lazy_workspace_step(z, leaves[2 + l], gm_[l], split=True)
            else:
                z, d = ops.lazy_workspace_step(z, leaves[2 + l], gm_[l])
                zb = z
            dl.append(d)
        out = torch.stack(dl).sum(0)  # a consumer of every dz, as the materialisation
        return torch.autograd.grad([out] + zs, leaves, [gm] + H)

    for a, b in zip(grads(True), grads(False)):
        assert torch.equal(a, b)


# ---------------------------------------------------------------------------
# configuration 5: 128x128 grid / 32x32 workspace, C=1024, L=24 (B=2 slice)
# ---------------------------------------------------------------------------
def test_config5_shape_bf16(coracle):
    B, G, C, L = 2, 32, 1024, 24
    d = cfg(B, G, C, L, grads=True)
    x0, g = dev(d["x0"], BF16), dev(d["grad_xl"], BF16)
    alpha, betas = dev(d["alpha"]), [dev(b) for b in d["beta"]]
    dzs = [dev(z, BF16) for z in d["dz"]]
    x0h, gh, dzh = host(x0), host(g), [host(z) for z in dzs]
    assert_bf16(host(capi.read(x0, alpha)), coracle.Cread(x0h, d["alpha"], G), what="read")
    assert_bf16(host(capi.materialise(x0, dzs, betas)), coracle.Cwrite(x0h, dzh, list(d["beta"])), what="materialise")
    ref = coracle.Cread_multi(gh, list(d["beta"]), G)
    for l, got in enumerate(capi.read_multi(g, betas)):
        assert_bf16(host(got), ref[l], what=f"gdZ_{l}")
    assert_f32(host(capi.weight_grad(g, dzs)), coracle.Cweight_grad(gh, dzh, G), what="gbeta")


def test_config5_full_batch_materialise_bf16(coracle):
    """Configuration 5 at its full batch (B=32: every grid step of the deep materialisation): samples 0, 17 and 31
    against the C oracle, and dZ = 0 giving X0 back bit for bit."""
    B, G, C, L = 32, 32, 1024, 24
    gen = torch.Generator(device=DEV).manual_seed(5)
    x0 = torch.randn((B, 4 * G, 4 * G, C), generator=gen, device=DEV).to(BF16)
    betas = [torch.randn((C, 16), generator=gen, device=DEV) * 0.02 for _ in range(L)]
    dzs = [(torch.randn((B, G * G, C), generator=gen, device=DEV) * 0.02).to(BF16) for _ in range(L)]
    out = capi.materialise(x0, dzs, betas)
    bh = [host(b) for b in betas]
    for b in (0, 17, B - 1):
        ref = coracle.Cwrite(host(x0[b : b + 1]), [host(z[b : b + 1]) for z in dzs], bh)
        assert_bf16(host(out[b : b + 1]), ref, what=f"materialise sample {b}")
    zeros = [torch.zeros_like(z) for z in dzs[:1]] * L
    assert torch.equal(capi.materialise(x0, zeros, betas), x0)


@pytest.mark.parametrize(
    "B,G,C,L,xdt,wdt",
    [
        (4, 16, 768, 12, BF16, F32),   # configuration 3's layer count and width, the fused pass
        (2, 16, 768, 5, BF16, F32),    # padded depth bucket (8)
        (2, 16, 128, 1, torch.float16, torch.float16),
        (2, 8, 64, 4, F32, F32),
        (1, 32, 1024, 12, BF16, BF16),  # configuration 5's grid and width
        (2, 16, 768, 13, BF16, F32),   # padded depth-24 bucket (8 wavefronts; the second block of 16 layers empty)
        (2, 16, 768, 18, torch.float16, torch.float16),  # the second block of 16 layers partly filled
        (1, 32, 1024, 24, BF16, F32),  # configuration 5's grid, width and depth
        (1, 8, 64, 25, BF16, F32),     # deeper than the fused kernel: the two separate passes
        (2, 4, 260, 3, BF16, F32),     # C not a multiple of 64: the two separate passes
    ],
)
def test_materialise_backward_fused_pass(coracle, B, G, C, L, xdt, wdt):
    """lthc_materialise_bwd: gdZ bitwise equal to lthc_read_multi_fwd, gbeta equal to lthc_weight_grad up to the
    summation order (same cells, partials grouped differently), both against the oracle."""
    print(f"case B={B} G={G} C={C} L={L} x={xdt} w={wdt}", flush=True)
    d = cfg(B, G, C, L, seed=L + C, grads=True)
    g = dev(d["grad_xl"], xdt)
    betas = [dev(b, wdt) for b in d["beta"]]
    dzs = [dev(z, xdt) for z in d["dz"]]
    gdz, gb = capi.materialise_bwd(g, dzs, betas)
    for l, (a, r) in enumerate(zip(gdz, capi.read_multi(g, betas))):
        assert torch.equal(a, r), f"gdZ_{l} differs from lthc_read_multi_fwd"
    sep = capi.weight_grad(g, dzs)
    assert_f32(host(gb), host(sep), tol=1e-5, what="gbeta vs lthc_weight_grad")
    gh, dzh = host(g), [host(z) for z in dzs]
    bh = [host(b) for b in betas]
    ref_dz = coracle.Cread_multi(gh, bh, G)
    for l in range(L):
        if xdt == F32:
            assert_f32(host(gdz[l]), ref_dz[l], what=f"gdZ_{l}")
        else:
            assert np.abs(host(gdz[l]) - ref_dz[l]).max() <= 2e-2 * max(1.0, np.abs(ref_dz[l]).max())
    assert_f32(host(gb), coracle.Cweight_grad(gh, dzh, G), tol=1e-5, what="gbeta")
    again = capi.materialise_bwd(g, dzs, betas)
    assert torch.equal(again[1], gb), "gbeta is not reproducible run to run"


def test_final_accumulate_backward_op_matches_reference_ops():
    """jit_thc::final_accumulate_backward equals the reference's two backward ops (gdZ bitwise, gbeta to 1e-5), and
    the 12-pointer op's autograd, which uses it, gives the same gradients."""
    B, G, C, L = 2, 16, 768, 12
    d = cfg(B, G, C, L, seed=21, grads=True)
    g = dev(d["grad_xl"], BF16)
    betas = [dev(b) for b in d["beta"]]
    dzs = [dev(z, BF16) for z in d["dz"]]
    gdz, gb = ops.final_accumulate_backward(g, dzs, betas)
    assert torch.equal(gdz, ops.final_accumulate_b4_12_grad_dz_ptr_traceable(g, *betas))
    ref_gb = ops.final_accumulate_b4_12_grad_beta_ptr_traceable(g, *dzs)
    assert_f32(host(gb), host(ref_gb), tol=1e-5, what="gbeta")
    x0 = dev(d["x0"], BF16).requires_grad_(True)
    bl = [b.clone().requires_grad_(True) for b in betas]
    zl = [z.clone().requires_grad_(True) for z in dzs]
    ops.final_accumulate_b4_12_traceable(x0, *zl, *bl).backward(g)
    assert torch.equal(x0.grad, g)
    for l in range(L):
        assert torch.equal(zl[l].grad, gdz[l])
        assert torch.equal(bl[l].grad, gb[l])


def test_config5_list_op_and_autograd_bf16(coracle):
    """jit_thc::final_accumulate_list at configuration 5's shape: forward, and its autograd (gdZ_l, gbeta_l)."""
    B, G, C, L = 2, 32, 1024, 24
    d = cfg(B, G, C, L, seed=4, grads=True)
    x0 = dev(d["x0"], BF16).requires_grad_(True)
    betas = [dev(b).requires_grad_(True) for b in d["beta"]]
    dzs = [dev(z, BF16).requires_grad_(True) for z in d["dz"]]
    xl = ops.final_accumulate_list(x0, dzs, betas)
    x0h, dzh = host(x0), [host(z) for z in dzs]
    assert_bf16(host(xl), coracle.Cwrite(x0h, dzh, list(d["beta"])), what="X_L")
    g = dev(d["grad_xl"], BF16)
    xl.backward(g)
    assert torch.equal(x0.grad, g)
    gh = host(g)
    ref_dz = coracle.Cread_multi(gh, list(d["beta"]), G)
    ref_beta = coracle.Cweight_grad(gh, dzh, G)
    for l in range(L):
        assert_bf16(host(dzs[l].grad), ref_dz[l], what=f"gdZ_{l}")
        assert_f32(host(betas[l].grad), ref_beta[l], tol=1e-5, what=f"gbeta_{l}")


# ---------------------------------------------------------------------------
# edge cases: ragged channel counts, every depth bucket, batch 1 and 0
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("B,G,C,L", [(1, 2, 4, 1), (3, 4, 260, 2), (1, 8, 12, 3), (2, 4, 36, 5), (1, 4, 20, 13), (1, 2, 8, 33), (1, 2, 8, 48)])
def test_edge_shapes_fp32(coracle, B, G, C, L):
    d = cfg(B, G, C, L, seed=B + G + C + L, grads=True)
    x0, g = dev(d["x0"]), dev(d["grad_xl"])
    betas, dzs = [dev(b) for b in d["beta"]], [dev(z) for z in d["dz"]]
    assert_f32(host(capi.read(x0, dev(d["alpha"]))), coracle.Cread(d["x0"], d["alpha"], G), what="read")
    assert_f32(host(capi.materialise(x0, dzs, betas)), coracle.Cwrite(d["x0"], list(d["dz"]), list(d["beta"])), what="materialise")
    ref = coracle.Cread_multi(d["grad_xl"], list(d["beta"]), G)
    for l, got in enumerate(capi.read_multi(g, betas)):
        assert_f32(host(got), ref[l], what=f"gdZ_{l}")
    assert_f32(host(capi.weight_grad(g, dzs)), coracle.Cweight_grad(d["grad_xl"], list(d["dz"]), G), what="gbeta")
    gam = capi.gamma(dev(d["alpha"]), betas)
    assert_f32(host(gam), coracle.Cgamma(d["alpha"], list(d["beta"])), tol=1e-6, what="gamma")


# Depths 17-24 with a base run the deep whole-cell kernel (the weights of layers 10 and up staged in LDS; with 8 | G
# two cells per wavefront and layers 4 and up in LDS): ragged channel slabs (C % 64 != 0), workspace grids that its
# 4 cells per block do not divide, padded depths (L < 24) and each activation / weight pair.
@pytest.mark.parametrize(
    "B,G,C,L,xdt,wdt",
    [(1, 2, 8, 17, F32, F32), (2, 6, 100, 24, BF16, F32), (1, 5, 68, 21, torch.float16, torch.float16),
     (2, 16, 256, 23, BF16, BF16), (3, 3, 192, 24, F32, F32), (1, 4, 64, 19, torch.float16, F32),
     (1, 8, 100, 24, BF16, F32), (2, 8, 72, 24, F32, F32)],
)  # fmt: skip
def test_deep_materialise(coracle, B, G, C, L, xdt, wdt):
    d = cfg(B, G, C, L, seed=B * G + C + L)
    x0 = dev(d["x0"], xdt)
    betas = [dev(b, wdt) for b in d["beta"]]
    dzs = [dev(z, xdt) for z in d["dz"]]
    got = host(capi.materialise(x0, dzs, betas))
    ref = coracle.Cwrite(host(x0), [host(z) for z in dzs], [host(b) for b in betas])
    if xdt == F32:
        assert_f32(got, ref, what="materialise")
    else:  # one rounding of the fp32 sum
        ulp = 2.0**-11 if xdt == torch.float16 else 2.0**-8
        err = np.abs(got - ref)
        assert (err <= ulp * np.abs(ref) + 1e-6).all(), f"rounding bound violated: {err.max()}"


@pytest.mark.parametrize("xdt,wdt", [(torch.float16, torch.float16), (torch.float16, F32), (BF16, BF16)])
def test_16bit_activations_and_weights(coracle, xdt, wdt):
    d = cfg(2, 16, 768, 3)
    x0 = dev(d["x0"], xdt)
    betas = [dev(b, wdt) for b in d["beta"]]
    dzs = [dev(z, xdt) for z in d["dz"]]
    got = host(capi.materialise(x0, dzs, betas))
    ref = coracle.Cwrite(host(x0), [host(z) for z in dzs], [host(b) for b in betas])
    ulp = 2.0**-11 if xdt == torch.float16 else 2.0**-8
    d_ = np.abs(got - ref)
    assert (d_ <= ulp * np.abs(ref) + 1e-6).all(), f"rounding bound violated: {d_.max()}"
    za = host(capi.read(x0, dev(d["alpha"], wdt)))
    zr = coracle.Cread(host(x0), rounded(d["alpha"], wdt), 16)
    assert (np.abs(za - zr) <= ulp * np.abs(zr) + 1e-5).all()
    # a pair without compiled kernels (fp16 activations, bf16 weights) goes through the op, which widens the weights
    if xdt == torch.float16:
        bb = torch.stack(betas).to(BF16)
        out = ops.final_accumulate_b4_traceable(x0, torch.stack(dzs), bb)
        ref2 = coracle.Cwrite(host(x0), [host(z) for z in dzs], [host(b) for b in bb])
        assert (np.abs(host(out) - ref2) <= ulp * np.abs(ref2) + 1e-6).all()


def test_empty_batch_and_misaligned_inputs():
    w = torch.full((8, 16), 1 / 16, device=DEV)
    z = ops.local_write_traceable(torch.empty(0, 16, 16, 8, device=DEV), w)
    assert z.shape == (0, 16, 8)
    gw = ops.local_weight_grad_traceable(torch.empty(0, 16, 16, 8, device=DEV), torch.empty(0, 16, 8, device=DEV))
    assert gw.shape == (8, 16) and float(gw.abs().max()) == 0.0
    base = torch.randn(1 + 16 * 16 * 8, device=DEV)
    x = base[1:].view(1, 16, 16, 8)  # storage offset of one element: misaligned for 16-byte vectors
    ref = ops.local_write_traceable(x.clone(), w)
    torch.testing.assert_close(ops.local_write_traceable(x, w), ref, rtol=0, atol=0)
    with pytest.raises(ValueError, match="multiple of 4"):
        ops.local_write_traceable(torch.randn(1, 16, 16, 6, device=DEV), torch.ones(6, 16, device=DEV))
    with pytest.raises(ValueError, match="cell side"):
        ops.local_write_traceable(torch.randn(1, 18, 18, 8, device=DEV), w)


# ---------------------------------------------------------------------------
# metric shape (B=256, C=768, L=12): size-independent properties
# ---------------------------------------------------------------------------
def test_metric_shape_properties_bf16():
    B, G, C, L = 256, 16, 768, 12
    gen = torch.Generator(device=DEV).manual_seed(0)
    x0 = torch.randn((B, 64, 64, C), generator=gen, device=DEV).to(BF16)
    alpha = torch.randn((C, 16), generator=gen, device=DEV) * 0.01 + 1 / 16
    betas = [torch.randn((C, 16), generator=gen, device=DEV) * 0.02 for _ in range(L)]
    dzs = [(torch.randn((B, 256, C), generator=gen, device=DEV) * 0.02).to(BF16) for _ in range(L)]
    # dZ == 0 leaves X0 bit-for-bit unchanged
    zeros = [torch.zeros_like(dzs[0])] * L
    assert torch.equal(capi.materialise(x0, zeros, betas), x0)
    # lazy invariant: read(X_L) == Z_L from the recurrence (bf16 rounding on both sides)
    xl = capi.materialise(x0, dzs, betas)
    z = capi.read(x0, alpha)
    gam = capi.gamma(alpha, betas)
    for l in range(L):
        z = capi.recur(z, dzs[l], gam[l])
    diff = (capi.read(xl, alpha).float() - z.float()).abs().max().item()
    assert diff <= 2e-2, f"R(X_L) vs Z_L: {diff}"
    # adjoint identity <R X, Zg> == <X, R^T Zg> in fp64 accumulation of fp32 kernel outputs
    xf = x0[:32].float()
    zg = dzs[0][:32].float()
    lhs = (capi.read(xf, alpha).double() * zg.double()).sum().item()
    rhs = (xf.double() * capi.materialise(None, [zg], [alpha]).double()).sum().item()
    assert abs(lhs - rhs) <= 1e-5 * max(1.0, abs(lhs))
    # checksum of checksums: sum_k gbeta_l[c,k] == sum_{b,m} dZ_l * read_{w=1}(G)
    gb = capi.weight_grad(x0, dzs[:2])
    ones = torch.ones((C, 16), device=DEV)
    r1 = capi.read(x0.float(), ones).double()
    for l in range(2):
        lhs = gb[l].double().sum(-1)
        rhs = (r1 * dzs[l].double()).sum((0, 1))
        assert ((lhs - rhs).abs().max() / rhs.abs().max()).item() <= 1e-5


def test_hip_graph_replay_matches_eager():
    B, G, C, L = 4, 16, 768, 12
    gen = torch.Generator(device=DEV).manual_seed(1)
    x0 = torch.randn((B, 64, 64, C), generator=gen, device=DEV).to(BF16)
    betas = [torch.randn((C, 16), generator=gen, device=DEV) * 0.02 for _ in range(L)]
    dzs = [(torch.randn((B, 256, C), generator=gen, device=DEV) * 0.02).to(BF16) for _ in range(L)]
    eager = ops.final_accumulate_b4_12_traceable(x0, *dzs, *betas)
    gb_eager = ops.final_accumulate_b4_12_grad_beta_ptr_traceable(x0, *dzs)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.final_accumulate_b4_12_traceable(x0, *dzs, *betas)  # warm the allocator on this stream
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.final_accumulate_b4_12_traceable(x0, *dzs, *betas)
        gb = ops.final_accumulate_b4_12_grad_beta_ptr_traceable(x0, *dzs)
    for i in range(3):
        out.zero_()
        gb.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        assert torch.equal(gb, gb_eager), f"replay {i}"



def test_interface_bwd_graph_replay_matches_eager():
    """lthc_interface_bwd (the single-pass tile kernel, the dalpha pass, the one-launch reductions and the gamma terms)
    captured in a HIP graph: every replay, with eager work and synchronisations between replays, equals the eager call
    bit for bit (the partial sums and counters need no clearing between calls)."""
    print("case interface_bwd graph replay", flush=True)
    B, G, C, L = 4, 16, 256, 12
    d = cfg(B, G, C, L, seed=91, grads=True)
    x0, alpha = dev(d["x0"], BF16), dev(d["alpha"])
    betas, dzs = [dev(b) for b in d["beta"]], [dev(z, BF16) for z in d["dz"]]
    gx = dev(d["grad_xl"], BF16)
    gzs = [None if l == 3 else dev(g, BF16) for l, g in enumerate(d["grad_z"])]
    eager = capi.interface_bwd(gx, gzs, x0, dzs, alpha, betas)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        capi.interface_bwd(gx, gzs, x0, dzs, alpha, betas)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = capi.interface_bwd(gx, gzs, x0, dzs, alpha, betas)
    flat = lambda r: [r[0], *r[1], r[2], r[3]]  # noqa: E731
    for i in range(3):
        other = capi.interface_bwd(gx, gzs, x0, [z * 0.5 for z in dzs], alpha, betas)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, ref in zip(flat(out), flat(eager)):
            assert torch.equal(got, ref), f"replay {i}"
        assert not torch.equal(other[2], eager[2])

# ---------------------------------------------------------------------------
# final-layer RMSNorm + modulate (jit_thc::norm_modulate, the materialisation's consumer)
# ---------------------------------------------------------------------------
def _eager_norm_modulate(x, w, shift, scale, eps=1e-6):
    """The reference's op sequence (jit_shared_adaln.py:26-30, local_thc.py:37-38) in torch."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    n = (xf * w).to(x.dtype)
    return n * (1 + scale.unsqueeze(1)) + shift.unsqueeze(1)


@pytest.mark.parametrize("dtype,C", [(F32, 768), (BF16, 768), (BF16, 1024), (F32, 260), (torch.float16, 768)])
def test_norm_modulate_forward_and_backward(dtype, C):
    g = torch.Generator().manual_seed(11)
    B, N = 3, 257
    x64 = torch.randn(B, N, C, generator=g, dtype=torch.float64)
    w64 = 1 + 0.1 * torch.randn(C, generator=g, dtype=torch.float64)
    sh64 = 0.2 * torch.randn(B, C, generator=g, dtype=torch.float64)
    sc64 = 0.2 * torch.randn(B, C, generator=g, dtype=torch.float64)
    gy64 = torch.randn(B, N, C, generator=g, dtype=torch.float64)
    x, sh, sc, gy = (t.to(DEV, dtype) for t in (x64, sh64, sc64, gy64))
    w = w64.to(DEV, F32)
    y, inv = ops.norm_modulate(x, w, sh, sc, 1e-6)
    ref_eager = _eager_norm_modulate(x, w, sh, sc)
    # exact function on the same (rounded) inputs in fp64, without intermediate roundings
    xd, wd, shd, scd = (t.double().cpu() for t in (x, w, sh, sc))
    inv64 = torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6)
    exact = (xd * inv64 * wd) * (1 + scd.unsqueeze(1)) + shd.unsqueeze(1)
    assert_f32(host(inv), inv64.reshape(-1).numpy(), tol=1e-6, what="inv")
    if dtype == F32:
        assert_f32(host(y), exact.numpy(), tol=1e-5, what="y fp32")
    else:  # no further from the exact function than the eager bf16 sequence itself
        err = (y.double().cpu() - exact).abs().max().item()
        err_eager = (ref_eager.double().cpu() - exact).abs().max().item()
        assert err <= 1.5 * err_eager + 1e-6, (err, err_eager)
        # the kernel performs the eager sequence's roundings: bit-identical but for rare one-ulp moves where the
        # fp32 mean is summed in another order
        same = (y == ref_eager).double().mean().item()
        assert same >= 0.99, f"only {same:.4f} of y is bit-identical to the eager sequence"
    # backward against torch autograd of the fp64 function
    xr, wr, shr, scr = (t.double().cpu().requires_grad_(True) for t in (x, w, sh, sc))
    inv_r = torch.rsqrt(xr.pow(2).mean(-1, keepdim=True) + 1e-6)
    yr = (xr * inv_r * wr) * (1 + scr.unsqueeze(1)) + shr.unsqueeze(1)
    yr.backward(gy.double().cpu())
    gx, gw, gsh, gsc = ops.norm_modulate_backward(gy, x, w, sc, inv)
    tol = 1e-5 if dtype == F32 else 1e-2
    assert_f32(host(gx), xr.grad.numpy(), tol=tol, what="dx")
    assert_f32(host(gw), wr.grad.numpy(), tol=max(tol, 1e-4), what="dweight")
    assert_f32(host(gsh), shr.grad.numpy(), tol=1e-5, what="dshift")
    assert_f32(host(gsc), scr.grad.numpy(), tol=max(tol, 1e-4), what="dscale")
    # the autograd registration returns the same gradients
    xa, wa, sha, sca = (t.clone().requires_grad_(True) for t in (x, w, sh, sc))
    ya, _ = ops.norm_modulate(xa, wa, sha, sca, 1e-6)
    ya.backward(gy)
    assert torch.equal(xa.grad, gx) and torch.equal(wa.grad, gw.to(wa.dtype))
    assert torch.equal(sha.grad, gsh.to(dtype)) and torch.equal(sca.grad, gsc.to(dtype))


# ---------------------------------------------------------------------------
# whole-interface entry points: recurrence prefix, read backward, interface fwd / bwd
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("xdt", [F32, BF16, torch.float16])
@pytest.mark.parametrize("C,L", [(768, 12), (768, 1), (260, 5)])
def test_recurrence_prefix_equals_single_steps(xdt, C, L):
    """lthc_recur_fwd_prefix: Z_1..Z_L bitwise equal to L lthc_recur_fwd launches (C = 260 takes the per-step
    path, the others the one-pass kernel), gamma fp32 or in the activation dtype."""
    print(f"case x={xdt} C={C} L={L}", flush=True)
    d = cfg(2, 16, C, L, seed=C + L, grads=True)
    z0 = dev(d["grad_z"][0] * 50.0, xdt)
    dzs = [dev(z, xdt) for z in d["dz"]]
    for gdt in (F32, xdt):
        gam = dev(np.stack([d["alpha"][:, l % 16] * 3.0 for l in range(L)]), gdt)
        got = capi.recur_prefix(z0, dzs, gam)
        z = z0
        for l in range(L):
            z = capi.recur(z, dzs[l], gam[l])
            assert torch.equal(got[l], z), f"Z_{l + 1} differs from the single steps"


def test_read_backward_entry():
    """lthc_read_bwd: dx = g_base + R^T gz (and without a base), dalpha = sum x gz, against the oracle (fp32)."""
    d = cfg(2, 16, 256, 1, seed=9, grads=True)
    x, gz, alpha, base = dev(d["x0"]), dev(d["grad_z"][0]), dev(d["alpha"]), dev(d["grad_xl"])
    dx, da = capi.read_bwd(gz, x, alpha, base)
    ref = O.write_np(d["grad_z"][0], d["alpha"], 64) + np.asarray(d["grad_xl"], np.float64)
    assert_f32(host(dx), ref, what="dx with base")
    assert_f32(host(da), O.weight_grad_np(d["x0"], d["grad_z"][0], 16), what="dalpha")
    dx0, _ = capi.read_bwd(gz, x, alpha)
    assert_f32(host(dx0), O.write_np(d["grad_z"][0], d["alpha"], 64), what="dx without base")


@pytest.mark.parametrize(
    "B,G,C,L,missing",
    [
        (2, 16, 64, 4, ()),
        (2, 16, 64, 4, (0,)),
        (2, 16, 64, 4, (2,)),
        (2, 16, 64, 4, (1, 2, 3)),
        # C % 64 != 0 and depth 26 > 24: the materialise backward and the recurrence prefix take their
        # per-layer fallbacks; an 8x8 workspace (32x32 grid) and a 32x32 one (128x128 grid)
        (1, 8, 72, 26, (5,)),
        (1, 32, 64, 2, ()),
    ],
)
def test_interface_entry_points_match_closed_form_fp32(B, G, C, L, missing):
    """lthc_interface_fwd against read / gamma / recurrence / materialise in float64, lthc_interface_bwd against the
    closed-form backward (oracle.interface_bwd_np); `missing` workspace gradients are passed as NULL (zero)."""
    print(f"case B={B} G={G} C={C} L={L} missing={missing}", flush=True)
    d = cfg(B, G, C, L, seed=17 + C + L, grads=True)
    x0, alpha = dev(d["x0"]), dev(d["alpha"])
    betas, dzs = [dev(b) for b in d["beta"]], [dev(z) for z in d["dz"]]
    zs, xl = capi.interface_fwd(x0, alpha, betas, dzs)
    z = O.read_np(d["x0"], d["alpha"], G)
    assert_f32(host(zs[0]), z, what="Z_0")
    for l in range(L):
        z = z + O.gamma_np(d["alpha"], d["beta"][l])[None, None, :] * np.asarray(d["dz"][l], np.float64)
        assert_f32(host(zs[l + 1]), z, what=f"Z_{l + 1}")
    xref = np.asarray(d["x0"], np.float64)
    for l in range(L):
        xref = xref + O.write_np(d["dz"][l], d["beta"][l], 4 * G)
    assert_f32(host(xl), xref, what="X_L")
    gz_np = [np.zeros_like(np.asarray(g)) if l in missing else g for l, g in enumerate(d["grad_z"])]
    gzs = [None if l in missing else dev(g) for l, g in enumerate(d["grad_z"])]
    dx0, ddz, da, db = capi.interface_bwd(dev(d["grad_xl"]), gzs, x0, dzs, alpha, betas)
    ref = O.interface_bwd_np(d["x0"], d["alpha"], list(d["dz"]), list(d["beta"]), d["grad_xl"], gz_np, G)
    assert_f32(host(dx0), ref["x0"], what="dX0")
    assert_f32(host(da), ref["alpha"], what="dalpha")
    for l in range(L):
        assert_f32(host(ddz[l]), ref["dz"][l], what=f"d dZ_{l}")
        assert_f32(host(db[l]), ref["beta"][l], what=f"dbeta_{l}")


@pytest.mark.parametrize("xdt", [BF16, torch.float16, F32])
@pytest.mark.parametrize(
    "L,missing,G",
    [(12, (), 16), (12, (0, 11), 16), (12, (3, 4, 5), 16), (5, (2,), 16), (24, (7,), 16), (3, (1, 2), 16),
     (12, (), 8), (24, (0,), 32)],  # one tile per cell row (G = 8); configuration 5's 32 x 32 workspace
)
def test_interface_bwd_one_pass_suffix_equals_per_step_chain(xdt, L, missing, G):
    """lthc_interface_bwd walks the recurrence backward of every step in one pass (recur_suffix_kernel, depth <= 24).
    Its dZ gradients and dX0 equal, bit for bit, the chain of per-step entry points it replaces: materialise
    backward, then l = L-1..0 one lthc_recur_bwd / lthc_recur_bwd_sum on the running suffix sum S_{l+1}, then
    S_0 = r(S_1 + H_0) and lthc_read_bwd.  The weight gradients sum in another order (relative 1e-5)."""
    print(f"case x={xdt} L={L} missing={missing} G={G}", flush=True)
    B, C = 2, 256
    d = cfg(B, G, C, L, seed=31 + L, grads=True)
    x0, alpha = dev(d["x0"], xdt), dev(d["alpha"])
    betas, dzs = [dev(b) for b in d["beta"]], [dev(z, xdt) for z in d["dz"]]
    gx = dev(d["grad_xl"], xdt)
    gzs = [None if l in missing else dev(g, xdt) for l, g in enumerate(d["grad_z"])]
    dx0, ddz, da, db = capi.interface_bwd(gx, gzs, x0, dzs, alpha, betas)

    gam = capi.gamma(alpha, betas)
    ref_dz, ref_db = capi.materialise_bwd(gx, dzs, betas)
    gg = [torch.zeros((C,), device=DEV) for _ in range(L)]
    cur = None
    for l in reversed(range(L)):
        h = gzs[l + 1] if l + 1 < L else None
        if cur is None and h is None:
            continue
        if cur is not None and h is not None:
            cur, ref_dz[l], gg[l] = capi.recur_bwd_sum(cur, h, dzs[l], gam[l], add=ref_dz[l])
        else:
            cur = cur if cur is not None else h
            ref_dz[l], gg[l] = capi.recur_bwd(cur, dzs[l], gam[l], add=ref_dz[l])
    if gzs[0] is not None:
        cur = gzs[0] if cur is None else (cur.float() + gzs[0].float()).to(xdt)
    assert cur is not None
    ref_dx0, ref_da = capi.read_bwd(cur, x0, alpha, gx)
    for l in range(L):
        assert torch.equal(ddz[l], ref_dz[l]), f"d dZ_{l}: {(ddz[l] != ref_dz[l]).float().mean().item():.2e} differ"
    assert torch.equal(dx0, ref_dx0)
    a = alpha.float()
    ref_da = ref_da + sum(gg[l][:, None] * betas[l] for l in range(L))
    ref_db = torch.stack([ref_db[l] + gg[l][:, None] * a for l in range(L)])
    for got, ref, what in ((da, ref_da, "dalpha"), (db, ref_db, "dbeta")):
        err = ((got - ref).abs().max() / ref.abs().max()).item()
        assert err <= 1e-5, f"{what}: {err:.3e}"



def test_interface_bwd_unaligned_x0_equals_aligned():
    """An X0 that is 8- but not 16-byte aligned: the tile kernel does not read X0 (dalpha's pass reads it with
    2-byte lanes), so lthc_interface_bwd gives the same dZ gradients and dX0 bit for bit, and the weight gradients
    to 1e-5."""
    print("case unaligned x0", flush=True)
    B, G, C, L = 2, 16, 256, 5
    d = cfg(B, G, C, L, seed=77, grads=True)
    x0 = dev(d["x0"], BF16)
    buf = torch.empty(x0.numel() + 4, dtype=BF16, device=DEV)
    x0u = buf[4:].view_as(x0)  # 8 bytes past a 16-byte boundary
    x0u.copy_(x0)
    assert x0u.data_ptr() % 16 == 8
    alpha, betas = dev(d["alpha"]), [dev(b) for b in d["beta"]]
    dzs, gx = [dev(z, BF16) for z in d["dz"]], dev(d["grad_xl"], BF16)
    gzs = [dev(g, BF16) for g in d["grad_z"]]
    got = capi.interface_bwd(gx, gzs, x0u, dzs, alpha, betas)
    ref = capi.interface_bwd(gx, gzs, x0, dzs, alpha, betas)
    assert torch.equal(got[0], ref[0]), "dX0"
    for l in range(L):
        assert torch.equal(got[1][l], ref[1][l]), f"d dZ_{l}"
    for g, r, what in ((got[2], ref[2], "dalpha"), (got[3], ref[3], "dbeta")):
        err = ((g - r).abs().max() / r.abs().max()).item()
        assert err <= 1e-5, f"{what}: {err:.3e}"

def _offset_views(ts):
    """Copies of `ts` whose storage starts 8 bytes past a 16-byte boundary (4-element aligned for 16-bit dtypes)."""
    out = []
    for t in ts:
        buf = torch.empty(t.numel() + 8 // t.element_size(), dtype=t.dtype, device=t.device)
        v = buf[8 // t.element_size() :].view_as(t)
        assert v.data_ptr() % 16 == 8
        out.append(v)
    return out


def test_tile_backward_outputs_8_bytes_off_equal_aligned():
    """The tile kernel writes gdZ / ddz with 16-byte stores, so outputs that are only 8-byte aligned (the ABI's
    4-element rule for bf16) must take the other kernels: lthc_materialise_bwd's gdZ and lthc_interface_bwd's ddz
    and dX0 then equal the aligned calls bit for bit, and the weight gradients agree to 1e-5."""
    print("case tile outputs 8 bytes off", flush=True)
    B, G, C, L = 2, 16, 256, 5
    d = cfg(B, G, C, L, seed=78, grads=True)
    x0, alpha = dev(d["x0"], BF16), dev(d["alpha"])
    betas, dzs = [dev(b) for b in d["beta"]], [dev(z, BF16) for z in d["dz"]]
    gx, gzs = dev(d["grad_xl"], BF16), [dev(g, BF16) for g in d["grad_z"]]
    lib, st = _abi.load(), torch.cuda.current_stream().cuda_stream
    # materialise backward
    ref_dz, ref_gb = capi.materialise_bwd(gx, dzs, betas)
    gdz = _offset_views(dzs)
    gb = torch.empty((L, C, 16), device=DEV)
    ws = torch.empty((int(lib.lthc_materialise_bwd_workspace_bytes(B, G, 4, C, L)) + 16,), device=DEV, dtype=torch.uint8)
    rc = lib.lthc_materialise_bwd(
        gx.data_ptr(), _abi.BF16, _abi.ptr_array(dzs), _abi.ptr_array(betas), _abi.F32, _abi.ptr_array(gdz),
        gb.data_ptr(), B, G, 4, C, L, ws.data_ptr(), ws.numel(), st,
    )  # fmt: skip
    _abi.check(rc, "lthc_materialise_bwd")
    for l in range(L):
        assert torch.equal(gdz[l], ref_dz[l]), f"gdZ_{l}"
    assert ((gb - ref_gb).abs().max() / ref_gb.abs().max()).item() <= 1e-5
    # whole-interface backward
    ref = capi.interface_bwd(gx, gzs, x0, dzs, alpha, betas)
    ddz = _offset_views(dzs)
    dx0 = torch.empty_like(x0)
    da = torch.empty((C, 16), device=DEV)
    db = torch.empty((L, C, 16), device=DEV)
    ws = torch.empty((int(lib.lthc_interface_workspace_bytes(B, G, 4, C, L)) + 16,), device=DEV, dtype=torch.uint8)
    rc = lib.lthc_interface_bwd(
        gx.data_ptr(), _abi.ptr_array(gzs), _abi.BF16, x0.data_ptr(), _abi.ptr_array(dzs), alpha.data_ptr(),
        _abi.ptr_array(betas), _abi.F32, dx0.data_ptr(), _abi.ptr_array(ddz), da.data_ptr(), db.data_ptr(),
        B, G, 4, C, L, ws.data_ptr(), ws.numel(), st,
    )  # fmt: skip
    _abi.check(rc, "lthc_interface_bwd")
    torch.cuda.synchronize()
    assert torch.equal(dx0, ref[0]), "dX0"
    for l in range(L):
        assert torch.equal(ddz[l], ref[1][l]), f"ddZ_{l}"
    for g, r, what in ((da, ref[2], "dalpha"), (db, ref[3], "dbeta")):
        err = ((g - r).abs().max() / r.abs().max()).item()
        assert err <= 1e-5, f"{what}: {err:.3e}"


def test_interface_entry_points_bf16_configuration3_slice(coracle):
    """The whole-interface entry points at configuration 3's width and depth (B=4 slice, bf16, fp32 weights):
    X_L within one bf16 rounding of the oracle, gradients to the bf16 bar."""
    B, G, C, L = 4, 16, 768, 12
    d = cfg(B, G, C, L, seed=23, grads=True)
    x0, alpha = dev(d["x0"], BF16), dev(d["alpha"])
    betas, dzs = [dev(b) for b in d["beta"]], [dev(z, BF16) for z in d["dz"]]
    zs, xl = capi.interface_fwd(x0, alpha, betas, dzs)
    x0h, dzh = host(x0), [host(z) for z in dzs]
    assert_bf16(host(xl), coracle.Cwrite(x0h, dzh, list(d["beta"])), what="X_L")
    assert_bf16(host(zs[0]), coracle.Cread(x0h, d["alpha"], G), what="Z_0")
    gx, gzs = dev(d["grad_xl"], BF16), [dev(g, BF16) for g in d["grad_z"]]
    dx0, ddz, da, db = capi.interface_bwd(gx, gzs, x0, dzs, alpha, betas)
    ref = O.interface_bwd_np(x0h, d["alpha"], dzh, list(d["beta"]), host(gx), [host(g) for g in gzs], G)
    assert np.abs(host(dx0) - ref["x0"]).max() <= 2e-2
    for l in range(L):
        assert np.abs(host(ddz[l]) - ref["dz"][l]).max() <= 2e-2, l
    # weight gradients sum bf16-rounded suffix sums over 1024 cells: relative to their scale
    for got, r, what in [(host(da), ref["alpha"], "dalpha")] + [(host(db[l]), ref["beta"][l], f"dbeta_{l}") for l in range(L)]:
        err = np.abs(got - r).max() / max(np.abs(r).max(), 1e-30)
        assert err <= 2e-2, f"{what}: {err:.3e}"


@pytest.mark.parametrize("xdt", [BF16, torch.float16])
@pytest.mark.parametrize(
    "B,G,C,L,wdt",
    [
        (2, 16, 768, 12, F32),   # configuration 3's width and depth: the one-pass kernel
        (2, 16, 256, 5, F32),    # padded depth bucket
        (1, 8, 512, 3, None),    # weights in the activation dtype
        (2, 4, 260, 3, F32),     # C not a multiple of 256: the composed form
        (1, 32, 256, 24, F32),   # configuration 5's depth and grid: the one-pass depth-24 kernel
        (2, 6, 100, 24, None),   # depth 24, ragged channel slab, grid not a multiple of 4 cells, 16-bit weights
        (2, 8, 192, 13, None),   # padded depths above 12: the composed form
    ],
)
def test_interface_fwd_one_pass_equals_per_op_chain(B, G, C, L, xdt, wdt):
    """lthc_interface_fwd reads X0 and each dZ_l once (iface_fwd_kernel, iface_fwd_deep_kernel at depth 24) where the
    shape allows it.  Z_0 .. Z_L and X_L equal, bit for bit, the per-op entry points it replaces: lthc_read_fwd,
    lthc_gamma (fp32), one lthc_recur_fwd per step and lthc_materialise_fwd."""
    wdt = wdt or xdt
    print(f"case B={B} G={G} C={C} L={L} x={xdt} w={wdt}", flush=True)
    d = cfg(B, G, C, L, seed=41 + L + C)
    x0, alpha = dev(d["x0"], xdt), dev(d["alpha"], wdt)  # alpha and the betas share the weight dtype
    betas, dzs = [dev(b, wdt) for b in d["beta"]], [dev(z, xdt) for z in d["dz"]]
    zs, xl = capi.interface_fwd(x0, alpha, betas, dzs)
    z = capi.read(x0, alpha)
    gam = capi.gamma(alpha, betas)
    assert torch.equal(zs[0], z), "Z_0 differs from lthc_read_fwd"
    for l in range(L):
        z = capi.recur(z, dzs[l], gam[l])
        assert torch.equal(zs[l + 1], z), f"Z_{l + 1} differs from the recurrence steps"
    assert torch.equal(xl, capi.materialise(x0, dzs, betas)), "X_L differs from lthc_materialise_fwd"
