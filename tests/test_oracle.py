"""Pins the CPU oracle (oracle/oracle.py, oracle/lthc_oracle.c) — CPU only.

The reference ships no tests or golden vectors for this path, so the oracle is
pinned by what the mathematics fixes:
  * brute-force loops over the explicit index map (tiny shapes);
  * library routines: depthwise F.conv2d / F.conv_transpose2d (stride = cell
    side, groups = C) — the equivalence the reference states at
    local_thc.py:620-692 — avg_pool2d (alpha = 1/16) and repeat_interleave
    (beta = 1) (local_thc.py:713-722);
  * the exact lazy identity R(X0 + sum_{j<l} P_j dZ_j) == Z0 + sum_{j<l} gamma_j dZ_j
    (docs/model.md:70-96);
  * torch.autograd through the conv-based forward for every backward formula.
Mutation tests plant plausible mistakes in copies of the oracle functions and
check that these checks catch them.
"""

import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O

RNG = np.random.default_rng(0)


def rand(*shape, scale=1.0):
    return RNG.standard_normal(shape) * scale


# ---------------------------------------------------------------------------
# library-routine forms (float64 torch, CPU)
# ---------------------------------------------------------------------------
def conv_read(x, alpha, g):
    """Depthwise strided conv2d == the channel-wise cell read."""
    xt = torch.as_tensor(x, dtype=torch.float64)
    b, h, _, c = xt.shape
    s = h // g
    w = torch.as_tensor(alpha, dtype=torch.float64).reshape(c, 1, s, s)
    out = F.conv2d(xt.permute(0, 3, 1, 2), w, stride=s, groups=c)
    return out.permute(0, 2, 3, 1).reshape(b, g * g, c)


def conv_write(dz, beta, h):
    """Depthwise strided conv_transpose2d == the channel-wise cell write."""
    dzt = torch.as_tensor(dz, dtype=torch.float64)
    b, m, c = dzt.shape
    g = int(round(m**0.5))
    s = h // g
    w = torch.as_tensor(beta, dtype=torch.float64).reshape(c, 1, s, s)
    out = F.conv_transpose2d(dzt.reshape(b, g, g, c).permute(0, 3, 1, 2), w, stride=s, groups=c)
    return out.permute(0, 2, 3, 1)


def loops_read(x, alpha, g):
    b, h, _, c = x.shape
    s = h // g
    z = np.zeros((b, g * g, c))
    for bb, m, k, cc in itertools.product(range(b), range(g * g), range(s * s), range(c)):
        z[bb, m, cc] += alpha[cc, k] * x[bb, (m // g) * s + k // s, (m % g) * s + k % s, cc]
    return z


def loops_write(dz, beta, h):
    b, m, c = dz.shape
    g = int(round(m**0.5))
    s = h // g
    x = np.zeros((b, h, h, c))
    for bb, mm, k, cc in itertools.product(range(b), range(m), range(s * s), range(c)):
        x[bb, (mm // g) * s + k // s, (mm % g) * s + k % s, cc] = beta[cc, k] * dz[bb, mm, cc]
    return x


# ---------------------------------------------------------------------------
# read / write
# ---------------------------------------------------------------------------
def test_read_matches_brute_force_loops():
    x, alpha = rand(2, 8, 8, 3), rand(3, 16)
    np.testing.assert_allclose(O.read_np(x, alpha, 2), loops_read(x, alpha, 2), rtol=1e-12, atol=1e-12)


def test_write_matches_brute_force_loops():
    dz, beta = rand(2, 4, 3), rand(3, 16)
    np.testing.assert_allclose(O.write_np(dz, beta, 8), loops_write(dz, beta, 8), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("b,g,c", [(2, 4, 8), (1, 16, 12), (3, 2, 5)])
def test_read_matches_depthwise_conv2d(b, g, c):
    x, alpha = rand(b, 4 * g, 4 * g, c), rand(c, 16)
    np.testing.assert_allclose(O.read_np(x, alpha, g), conv_read(x, alpha, g).numpy(), rtol=1e-12, atol=1e-12)


def test_read_uniform_alpha_is_avg_pool():
    x = rand(2, 16, 16, 6)
    alpha = np.full((6, 16), 1.0 / 16.0)
    ref = F.avg_pool2d(torch.as_tensor(x).permute(0, 3, 1, 2), kernel_size=4, stride=4)
    ref = ref.permute(0, 2, 3, 1).reshape(2, 16, 6).numpy()
    np.testing.assert_allclose(O.read_np(x, alpha, 4), ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("b,g,c", [(2, 4, 8), (1, 16, 12)])
def test_write_matches_depthwise_conv_transpose2d(b, g, c):
    dz, beta = rand(b, g * g, c), rand(c, 16)
    np.testing.assert_allclose(O.write_np(dz, beta, 4 * g), conv_write(dz, beta, 4 * g).numpy(), rtol=1e-12, atol=1e-12)


def test_write_unit_beta_is_nearest_upsample():
    dz = rand(2, 16, 5)
    ref = torch.as_tensor(dz).reshape(2, 4, 4, 5).repeat_interleave(4, 1).repeat_interleave(4, 2).numpy()
    np.testing.assert_allclose(O.write_np(dz, np.ones((5, 16)), 16), ref, rtol=0, atol=0)


def test_read_write_adjoint_identity():
    """<R X, Z> == <X, R^T Z>, and R^T is the write with the read weights."""
    x, alpha, z = rand(2, 16, 16, 7), rand(7, 16), rand(2, 16, 7)
    lhs = (O.read_np(x, alpha, 4) * z).sum()
    rhs = (x * O.write_np(z, alpha, 16)).sum()
    assert abs(lhs - rhs) <= 1e-10 * max(1.0, abs(lhs))


# ---------------------------------------------------------------------------
# gamma, lazy recurrence, materialisation
# ---------------------------------------------------------------------------
def test_gamma_is_read_of_write():
    """R(P_l(dZ)) == gamma_l * dZ exactly (docs/model.md:86-94)."""
    dz, alpha, beta = rand(2, 16, 9), rand(9, 16), rand(9, 16)
    lhs = O.read_np(O.write_np(dz, beta, 16), alpha, 4)
    np.testing.assert_allclose(lhs, O.gamma_np(alpha, beta)[None, None, :] * dz, rtol=1e-12, atol=1e-13)


def test_lazy_recurrence_equals_naive_reads():
    """Z_l of the lazy recurrence equals the read of the materialised X_l, for every l."""
    L, g, c = 5, 4, 6
    x0, alpha = rand(2, 4 * g, 4 * g, c), rand(c, 16) * 0.1 + 1 / 16
    betas = [rand(c, 16) for _ in range(L)]
    dzs = [rand(2, g * g, c) for _ in range(L)]
    zs, xl = O.lazy_forward_np(x0, alpha, dzs, betas, g)
    x = x0
    for l in range(L + 1):
        np.testing.assert_allclose(zs[l], conv_read(x, alpha, g).numpy(), rtol=1e-10, atol=1e-11)
        if l < L:
            x = x + conv_write(dzs[l], betas[l], 4 * g).numpy()
    np.testing.assert_allclose(xl, x, rtol=1e-12, atol=1e-12)


def _triangular_case(L=4, g=4, c=6, seed=3):
    rng = np.random.default_rng(seed)
    x0 = rng.standard_normal((2, 4 * g, 4 * g, c))
    alphas = [rng.standard_normal((c, 16)) * 0.1 + 1 / 16 for _ in range(L)]
    betas = [rng.standard_normal((c, 16)) for _ in range(L)]
    dzs = [rng.standard_normal((2, g * g, c)) for _ in range(L)]
    return x0, alphas, betas, dzs, g


def _naive_nonshared_reads(x0, alphas, betas, dzs, g):
    """z_l = R_l(X_{l}) of the materialised stream X_l = X0 + sum_{j<l} P_j dZ_j (depthwise convs)."""
    x, zs = x0, []
    for l in range(len(alphas)):
        zs.append(conv_read(x, alphas[l], g).numpy())
        x = x + conv_write(dzs[l], betas[l], 4 * g).numpy()
    return zs, x


def test_gamma_matrix_is_read_of_write():
    """gamma[l, j] * dZ == R_l(P_j(dZ)) for every (l, j), including l != j."""
    _, alphas, betas, dzs, g = _triangular_case(L=3)
    gam = O.gamma_matrix_np(alphas, betas)
    for l in range(3):
        for j in range(3):
            lhs = conv_read(conv_write(dzs[0], betas[j], 4 * g), alphas[l], g).numpy()
            np.testing.assert_allclose(lhs, gam[l, j][None, None, :] * dzs[0], rtol=1e-10, atol=1e-12)


def test_triangular_lazy_equals_naive_nonshared_reads():
    """The non-shared lazy schedule (separate R_l, P_j per layer) reproduces the naive high-res recurrence."""
    x0, alphas, betas, dzs, g = _triangular_case(L=5)
    zs, xl = O.triangular_lazy_np(x0, alphas, betas, dzs, g)
    ref_zs, ref_x = _naive_nonshared_reads(x0, alphas, betas, dzs, g)
    for l in range(5):
        np.testing.assert_allclose(zs[l], ref_zs[l], rtol=1e-10, atol=1e-11, err_msg=f"layer {l}")
    np.testing.assert_allclose(xl, ref_x, rtol=1e-12, atol=1e-12)


def test_mutation_triangular_off_by_one_is_caught():
    """Summing j <= l (the diagonal) or j < l - 1 (a dropped term) breaks the identity above."""
    x0, alphas, betas, dzs, g = _triangular_case(L=4)
    gam = O.gamma_matrix_np(alphas, betas)
    ref_zs, _ = _naive_nonshared_reads(x0, alphas, betas, dzs, g)
    base = conv_read(x0, alphas[2], g).numpy()
    assert not np.allclose(O.triangular_np(base, dzs[:3], gam[2]), ref_zs[2])
    assert not np.allclose(O.triangular_np(base, dzs[:1], gam[2]), ref_zs[2])
    assert not np.allclose(O.triangular_np(base, dzs[:2], gam[:, 2]), ref_zs[2])  # transposed gamma


def test_materialise_zero_updates_is_identity():
    x0 = rand(1, 8, 8, 4)
    out = O.final_accumulate_np(x0, [np.zeros((1, 4, 4))] * 3, [rand(4, 16) for _ in range(3)])
    np.testing.assert_array_equal(out, x0)


# ---------------------------------------------------------------------------
# backward formulas against torch.autograd of the conv-based forward
# ---------------------------------------------------------------------------
def _autograd_interface(x0, alpha, dzs, betas, grad_xl, grad_zs, g):
    """Naive forward with library ops: X_{l+1} = X_l + convT(dZ_l), Z_l = conv(X_l)."""
    t = lambda a: torch.tensor(np.asarray(a), dtype=torch.float64, requires_grad=True)  # noqa: E731
    x0_t, a_t = t(x0), t(alpha)
    b_t = [t(b) for b in betas]
    d_t = [t(d) for d in dzs]
    h = x0.shape[1]
    c = x0.shape[3]
    s = h // g
    x = x0_t
    loss = 0.0
    for l in range(len(dzs)):
        z = F.conv2d(x.permute(0, 3, 1, 2), a_t.reshape(c, 1, s, s), stride=s, groups=c)
        z = z.permute(0, 2, 3, 1).reshape(x.shape[0], g * g, c)
        loss = loss + (z * torch.as_tensor(grad_zs[l])).sum()
        w = F.conv_transpose2d(d_t[l].reshape(-1, g, g, c).permute(0, 3, 1, 2), b_t[l].reshape(c, 1, s, s), stride=s, groups=c)
        x = x + w.permute(0, 2, 3, 1)
    loss = loss + (x * torch.as_tensor(grad_xl)).sum()
    loss.backward()
    return {"x0": x0_t.grad.numpy(), "alpha": a_t.grad.numpy(), "dz": [d.grad.numpy() for d in d_t], "beta": [b.grad.numpy() for b in b_t]}


def _interface_case(L=4, g=4, c=6, b=2, seed=1):
    rng = np.random.default_rng(seed)
    r = lambda *s: rng.standard_normal(s)  # noqa: E731
    return dict(
        x0=r(b, 4 * g, 4 * g, c), alpha=r(c, 16) * 0.1 + 1 / 16, betas=[r(c, 16) for _ in range(L)],
        dzs=[r(b, g * g, c) for _ in range(L)], grad_xl=r(b, 4 * g, 4 * g, c), grad_zs=[r(b, g * g, c) for _ in range(L)], g=g,
    )  # fmt: skip


def test_interface_backward_matches_autograd():
    cs = _interface_case()
    ref = _autograd_interface(cs["x0"], cs["alpha"], cs["dzs"], cs["betas"], cs["grad_xl"], cs["grad_zs"], cs["g"])
    got = O.interface_bwd_np(cs["x0"], cs["alpha"], cs["dzs"], cs["betas"], cs["grad_xl"], cs["grad_zs"], cs["g"])
    np.testing.assert_allclose(got["x0"], ref["x0"], rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(got["alpha"], ref["alpha"], rtol=1e-10, atol=1e-10)
    for l in range(len(cs["dzs"])):
        np.testing.assert_allclose(got["dz"][l], ref["dz"][l], rtol=1e-10, atol=1e-10)
        np.testing.assert_allclose(got["beta"][l], ref["beta"][l], rtol=1e-10, atol=1e-10)


def test_weight_grad_and_read_multi_match_autograd_of_materialise():
    """gbeta_l and gdZ_l of X_L = X0 + sum P_l dZ_l (the materialise op's backward)."""
    L, g, c = 3, 4, 5
    x0, grad = rand(2, 16, 16, c), rand(2, 16, 16, c)
    betas = [rand(c, 16) for _ in range(L)]
    dzs = [rand(2, 16, c) for _ in range(L)]
    b_t = [torch.tensor(b, requires_grad=True) for b in betas]
    d_t = [torch.tensor(d, requires_grad=True) for d in dzs]
    x = torch.as_tensor(x0)
    for l in range(L):
        w = F.conv_transpose2d(d_t[l].reshape(2, g, g, c).permute(0, 3, 1, 2), b_t[l].reshape(c, 1, 4, 4), stride=4, groups=c)
        x = x + w.permute(0, 2, 3, 1)
    (x * torch.as_tensor(grad)).sum().backward()
    for l in range(L):
        np.testing.assert_allclose(O.weight_grad_np(grad, dzs[l], g), b_t[l].grad.numpy(), rtol=1e-10, atol=1e-10)
        np.testing.assert_allclose(O.read_np(grad, betas[l], g), d_t[l].grad.numpy(), rtol=1e-10, atol=1e-10)


def test_gradcheck_conv_forward_tiny():
    """torch.autograd.gradcheck of the library forms the backward checks rely on."""
    x = torch.randn(1, 8, 8, 2, dtype=torch.float64, requires_grad=True)
    a = torch.randn(2, 16, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda x_, a_: conv_read(x_, a_, 2), (x, a))
    z = torch.randn(1, 4, 2, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda z_, b_: conv_write(z_, b_, 8), (z, a))


def test_recurrence_backward_matches_autograd():
    z, dz, gam, gr = rand(2, 16, 8), rand(2, 16, 8), rand(8), rand(2, 16, 8)
    d_t, g_t = torch.tensor(dz, requires_grad=True), torch.tensor(gam, requires_grad=True)
    (torch.as_tensor(z) + g_t * d_t).mul(torch.as_tensor(gr)).sum().backward()
    np.testing.assert_allclose(gam * gr, d_t.grad.numpy(), rtol=1e-12)
    np.testing.assert_allclose((gr * dz).sum((0, 1)), g_t.grad.numpy(), rtol=1e-12)


# ---------------------------------------------------------------------------
# the C restatement against the numpy one
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("b,g,c,L", [(2, 4, 12, 3), (1, 8, 20, 1), (2, 2, 4, 5)])
def test_c_oracle_matches_numpy(coracle, b, g, c, L):
    rng = np.random.default_rng(b * 100 + g * 10 + c)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    h = 4 * g
    x, alpha = f(b, h, h, c), f(c, 16)
    betas, dzs = [f(c, 16) for _ in range(L)], [f(b, g * g, c) for _ in range(L)]
    tol = dict(rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(coracle.Cread(x, alpha, g), O.read_np(x, alpha, g), **tol)
    np.testing.assert_allclose(coracle.Cwrite(x, dzs, betas), O.final_accumulate_np(x, dzs, betas), **tol)
    np.testing.assert_allclose(coracle.Cwrite(None, dzs[:1], betas[:1], h=h), O.write_np(dzs[0], betas[0], h), **tol)
    for got, w in zip(coracle.Cread_multi(x, betas, g), betas, strict=True):
        np.testing.assert_allclose(got, O.read_np(x, w, g), **tol)
    gw = coracle.Cweight_grad(x, dzs, g)
    for l in range(L):
        np.testing.assert_allclose(gw[l], O.weight_grad_np(x, dzs[l], g), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(coracle.Cgamma(alpha, betas), np.stack([O.gamma_np(alpha, bt) for bt in betas]), **tol)
    gam = f(c)
    np.testing.assert_allclose(coracle.Crecur(dzs[0], dzs[-1], gam), O.lazy_update_np(dzs[0], dzs[-1], gam), **tol)
    gdz, gg = coracle.Crecur_bwd(dzs[0], dzs[-1], gam)
    np.testing.assert_allclose(gdz, gam * dzs[0], **tol)
    np.testing.assert_allclose(gg, (dzs[0].astype(np.float64) * dzs[-1]).sum((0, 1)), rtol=1e-5, atol=1e-5)


def test_c_oracle_thread_count_invariant(coracle):
    x, lo = RNG.standard_normal((2, 16, 16, 24)).astype(np.float32), RNG.standard_normal((2, 16, 24)).astype(np.float32)
    n = coracle.max_threads()
    coracle.set_threads(1)
    a = coracle.Cweight_grad(x, [lo], 4)
    coracle.set_threads(max(2, n))
    b = coracle.Cweight_grad(x, [lo], 4)
    coracle.set_threads(n)
    np.testing.assert_array_equal(a, b)


def test_seeded_inputs_are_reproducible():
    a = O.make_inputs(1, 2, 8, 2, seed=0, grads=True)
    b = O.make_inputs(1, 2, 8, 2, seed=0, grads=True)
    for k in a:
        np.testing.assert_array_equal(a[k], b[k])
    big = O.make_inputs(2, 16, 768, 1, seed=0)
    assert abs(big["alpha"].mean() - 1 / 16) < 1e-3 and abs(big["alpha"].std() - 0.01) < 1e-3
    assert abs(big["beta"].std() - 0.02) < 1e-3 and abs(big["x0"].std() - 1.0) < 1e-2


# ---------------------------------------------------------------------------
# mutation tests: plausible oracle mistakes are caught by the checks above
# ---------------------------------------------------------------------------
def test_mutation_swapped_tap_axes_is_caught():
    x, alpha = rand(2, 16, 16, 16), rand(16, 16)
    swapped = alpha.reshape(16, 4, 4).transpose(0, 2, 1).reshape(16, 16)  # sy <-> sx
    assert not np.allclose(O.read_np(x, swapped, 4), conv_read(x, alpha, 4).numpy())
    assert not np.allclose(O.write_np(rand(2, 16, 16), swapped, 16)[0], 0)  # non-degenerate
    dz = rand(2, 16, 16)
    assert not np.allclose(O.write_np(dz, swapped, 16), conv_write(dz, alpha, 16).numpy())


def test_mutation_transposed_weight_is_caught():
    x, alpha = rand(2, 16, 16, 16), rand(16, 16)  # C == K, so [K,C] has the same shape
    assert not np.allclose(O.read_np(x, alpha.T, 4), conv_read(x, alpha, 4).numpy())


def test_mutation_dropped_layer_is_caught():
    x0 = rand(1, 8, 8, 4)
    betas, dzs = [rand(4, 16) for _ in range(3)], [rand(1, 4, 4) for _ in range(3)]
    dropped = O.final_accumulate_np(x0, dzs[:-1], betas[:-1])
    x = x0 + sum(conv_write(d, b, 8).numpy() for d, b in zip(dzs, betas))
    assert not np.allclose(dropped, x)


def test_mutation_wrong_sign_in_backward_is_caught():
    cs = _interface_case(L=2)
    ref = _autograd_interface(cs["x0"], cs["alpha"], cs["dzs"], cs["betas"], cs["grad_xl"], cs["grad_zs"], cs["g"])
    got = O.interface_bwd_np(cs["x0"], cs["alpha"], cs["dzs"], cs["betas"], cs["grad_xl"], [-gz for gz in cs["grad_zs"]], cs["g"])
    assert not np.allclose(got["dz"][0], ref["dz"][0])
    assert not np.allclose(got["alpha"], ref["alpha"])


def test_torch_cpu_sequence_matches_numpy_oracle():
    """oracle/torch_cpu.py (the reference's eager op sequence, timed as the CPU baseline) equals the numpy oracle's
    read, gamma, recurrence and materialisation, which the depthwise-convolution and brute-force checks above pin."""
    import torch

    from oracle import torch_cpu as TC

    B, G, C, L = 2, 4, 12, 3
    d = O.make_inputs(B, G, C, L, seed=5)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).double()  # noqa: E731
    x0, alpha = t(d["x0"]), t(d["alpha"])
    betas, dzs = [t(b) for b in d["beta"]], [t(z) for z in d["dz"]]
    np.testing.assert_allclose(TC.read(x0, alpha, G).numpy(), O.read_np(d["x0"], d["alpha"], G), rtol=1e-12, atol=1e-12)
    for l in range(L):
        np.testing.assert_allclose(TC.gamma(alpha, betas[l]).numpy(), O.gamma_np(d["alpha"], d["beta"][l]), rtol=1e-12)
    zl, xl = TC.step(x0, alpha, betas, dzs, G)
    z_ref = O.read_np(d["x0"], d["alpha"], G)
    for l in range(L):
        z_ref = O.lazy_update_np(z_ref, d["dz"][l], O.gamma_np(d["alpha"], d["beta"][l]))
    np.testing.assert_allclose(zl.numpy(), z_ref, rtol=1e-12, atol=1e-12)
    xl_ref = O.final_accumulate_np(d["x0"], list(d["dz"]), list(d["beta"]))
    np.testing.assert_allclose(xl.numpy(), xl_ref, rtol=1e-12, atol=1e-12)
    # the lazy identity holds through this sequence too: R(X_L) == Z_L
    np.testing.assert_allclose(TC.read(xl, alpha, G).numpy(), zl.numpy(), rtol=1e-10, atol=1e-10)
