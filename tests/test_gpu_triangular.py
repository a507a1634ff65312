"""GPU parity of the non-shared (triangular lazy) interface ops against the CPU oracle (MI355X only).

Ops: ``jit_thc::triangular_accumulate_traceable`` / ``_list`` / ``_b4_12_ptr_traceable`` /
``_b4_12_ptr_active[N]`` (workspace accumulation, ``lthc_ws_accumulate_*``) and
``jit_thc::all_base_b4_12[_split]_traceable`` (per-layer bases R_l(x0), ``lthc_read_multi_fwd``,
with gradients through ``lthc_materialise_fwd`` without a base and ``lthc_weight_grad``).
Tolerances are those of test_gpu_parity: fp32 max|d|/max|ref| <= 1e-5; bf16 max|d| <= 2e-2 and
|d| <= 2^-8|ref| + 1e-5 against the fp64 oracle on the same bf16-rounded inputs.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from flowmatching_lthc_amd import ops_triangular as T
from oracle import oracle as O

from .test_gpu_parity import BF16, DEV, F32, assert_bf16, assert_f32, dev, host, rounded

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _oracle_built(coracle):
    coracle.set_threads(16)
    yield


def ws_case(B, G, C, L, seed=0):
    gen = torch.Generator().manual_seed(seed)
    base = torch.randn((B, G * G, C), generator=gen)
    dzs = torch.randn((L, B, G * G, C), generator=gen) * 0.02
    gamma = torch.randn((L, C), generator=gen) * 0.1 + 1.0
    grad = torch.randn((B, G * G, C), generator=gen) * 1e-3
    return base.numpy(), dzs.numpy(), gamma.numpy(), grad.numpy()


def check(got, ref, dtype, what):
    (assert_f32 if dtype == F32 else assert_bf16)(got, ref, what=what)


# ---------------------------------------------------------------------------
# stacked and list forms, every depth bucket
# ---------------------------------------------------------------------------
@pytest.mark.parametrize(
    "dt,gdt,B,G,C,L",
    [
        (F32, F32, 2, 16, 768, 1),
        (F32, F32, 2, 4, 260, 5),
        (BF16, BF16, 4, 16, 768, 12),
        (BF16, F32, 2, 8, 1024, 13),
        (F32, F32, 1, 4, 36, 24),
        (BF16, BF16, 1, 4, 12, 7),
        # the one-thread-per-run forward with two rows per thread (16-bit activations, fp32 gamma): even rows, and
        # 27 rows, whose last thread has one row; then one row per thread in fp32 with an odd row count
        (BF16, F32, 2, 16, 768, 4),
        (BF16, F32, 3, 3, 768, 11),
        (F32, F32, 1, 3, 64, 3),
    ],
)
def test_triangular_stacked_and_list_forward_backward(dt, gdt, B, G, C, L):
    print(f"case dt={dt} gamma={gdt} B={B} G={G} C={C} L={L}", flush=True)
    base, dzs, gamma, grad = ws_case(B, G, C, L, seed=L)
    rb, rd, rg, rgr = rounded(base, dt), rounded(dzs, dt), rounded(gamma, gdt), rounded(grad, dt)
    ref = O.triangular_np(rb, list(rd), rg)

    tb, td, tg = dev(base, dt).requires_grad_(), dev(dzs, dt).requires_grad_(), dev(gamma, gdt).requires_grad_()
    out = T.triangular_accumulate_traceable(tb, td, tg)
    assert out.dtype == dt and out.shape == tb.shape
    check(host(out), ref, dt, "forward")
    out.backward(dev(grad, dt))
    assert torch.equal(tb.grad, dev(grad, dt)), "grad_base is grad_out"
    for l in range(L):
        check(host(td.grad[l]), rg[l][None, None, :] * rgr, dt, f"gdz[{l}]")
    gg_ref = np.einsum("bmc,lbmc->lc", rgr.astype(np.float64), rd.astype(np.float64))
    assert tg.grad.dtype == gdt
    check(host(tg.grad), gg_ref, gdt, "ggamma")

    # the list form is the same kernel: identical bits, also through autograd
    lb = dev(base, dt).requires_grad_()
    ld = [dev(d, dt).requires_grad_() for d in dzs]
    lg = dev(np.concatenate([gamma, gamma[:1]], 0), gdt).requires_grad_()  # one extra, unused row
    out2 = T.triangular_accumulate_list(lb, ld, lg)
    assert torch.equal(out2, out.detach())
    out2.backward(dev(grad, dt))
    for l in range(L):
        assert torch.equal(ld[l].grad, td.grad[l])
    assert torch.equal(lg.grad[:L], tg.grad) and not lg.grad[L].any()


@pytest.mark.parametrize("gdt,rows,L", [(BF16, 512, 11), (F32, 512, 11), (F32, 27, 5), (BF16, 27, 2)])
def test_triangular_forward_kernels_bitwise_equal(gdt, rows, L):
    """The forward's two kernels give the same bits: 16-byte aligned operands take the one-thread-per-run kernel,
    operands 8 bytes off a 16-byte boundary (the ABI's 4-element rule still holds) the grid-stride kernel."""
    print(f"case forward kernels gamma={gdt} rows={rows} L={L}", flush=True)
    C = 768
    gen = torch.Generator(device=DEV).manual_seed(rows + L)

    def tensors(shift):  # bf16 [rows, C] views starting `shift` elements into their buffers
        def one(scale):
            buf = torch.empty(rows * C + 8, device=DEV, dtype=BF16)
            v = buf[shift : shift + rows * C].view(1, rows, C)
            v.copy_((torch.randn((1, rows, C), generator=gen, device=DEV) * scale).to(BF16))
            return v

        return one(1.0), [one(0.02) for _ in range(L)]

    gamma = (torch.randn((L, C), generator=gen, device=DEV) * 0.1 + 1.0).to(gdt)
    base, dzs = tensors(0)
    base2, dzs2 = tensors(4)
    base2.copy_(base)
    for a, b in zip(dzs2, dzs):
        a.copy_(b)
    assert base.data_ptr() % 16 == 0 and base2.data_ptr() % 16 == 8
    flat = T.triangular_accumulate_list(base, dzs, gamma)
    strided = T.triangular_accumulate_list(base2, dzs2, gamma)
    assert torch.equal(flat, strided)


def test_triangular_grad_ops_direct():
    base, dzs, gamma, grad = ws_case(2, 16, 768, 3, seed=5)
    g, gm, dzt = dev(grad, BF16), dev(gamma, BF16), dev(dzs, BF16)
    gdz = torch.ops.jit_thc.triangular_accumulate_grad_dz(g, gm)
    assert gdz.shape == (3, 2, 256, 768) and gdz.dtype == BF16
    for l in range(3):
        assert_bf16(host(gdz[l]), rounded(gamma, BF16)[l][None, None, :] * rounded(grad, BF16), what=f"gdz{l}")
    gg = torch.ops.jit_thc.triangular_accumulate_grad_gamma(g, dzt, gm)
    assert gg.dtype == F32 and gg.shape == (3, 768)
    ref = np.einsum("bmc,lbmc->lc", rounded(grad, BF16).astype(np.float64), rounded(dzs, BF16).astype(np.float64))
    assert_f32(host(gg), ref, what="ggamma")


def test_triangular_rejects_bad_shapes():
    base, dzs, gamma, _ = ws_case(1, 4, 8, 2)
    tb, td, tg = dev(base), dev(dzs), dev(gamma)
    with pytest.raises(ValueError):
        T.triangular_accumulate_list(tb, [td[0]] * 25, dev(np.ones((25, 8), np.float32)))
    with pytest.raises(ValueError):
        T.triangular_accumulate_list(tb, [td[0], td[1]], tg[:1])
    with pytest.raises(ValueError):
        T.triangular_accumulate_list(tb, [td[0][:, :8]], tg)
    with pytest.raises(ValueError):
        T.triangular_accumulate_list(dev(np.zeros((1, 16, 6), np.float32)), [dev(np.zeros((1, 16, 6), np.float32))], dev(np.ones((1, 6), np.float32)))


# ---------------------------------------------------------------------------
# 12-pointer and active-prefix ops
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("active", [1, 5, 11])
def test_tri12_active_ops_forward_backward(active):
    print(f"case active={active}", flush=True)
    base, dzs, gamma, grad = ws_case(2, 16, 768, 12, seed=active)
    rb, rd, rg, rgr = (rounded(a, BF16) for a in (base, dzs, gamma, grad))
    ref = O.triangular_np(rb, list(rd[:active]), rg)

    def leaves():
        return dev(base, BF16).requires_grad_(), [dev(d, BF16).requires_grad_() for d in dzs], dev(gamma, BF16).requires_grad_()

    tb, td, tg = leaves()
    out = torch.ops.jit_thc.triangular_accumulate_b4_12_ptr_active(tb, *td, tg, active)
    assert_bf16(host(out), ref, what="active forward")
    out.backward(dev(grad, BF16))
    for j in range(12):
        if j < active:
            assert_bf16(host(td[j].grad), rg[j][None, None, :] * rgr, what=f"gdz{j}")
        else:
            assert td[j].grad is None, f"dz{j} beyond the active prefix got a gradient"
    gg_ref = np.einsum("bmc,lbmc->lc", rgr.astype(np.float64), rd[:active].astype(np.float64))
    assert_bf16(host(tg.grad[:active]), gg_ref, what="ggamma")
    assert not tg.grad[active:].any()

    # the op with the prefix in its name (the reference's list of 11 ops) gives the same bits
    tb2, td2, tg2 = leaves()
    out2 = T.triangular_accumulate_b4_12_ptr_active_traceable_ops[active - 1](tb2, *td2, tg2)
    assert torch.equal(out2, out.detach())
    out2.backward(dev(grad, BF16))
    assert torch.equal(tg2.grad, tg.grad)
    assert all((td2[j].grad is None) == (td[j].grad is None) for j in range(12))

    gdz = torch.ops.jit_thc.triangular_accumulate_b4_12_ptr_active_grad_dz(dev(grad, BF16), dev(gamma, BF16), active)
    assert gdz.shape[0] == active


def test_tri12_all_layers_and_active_bounds():
    base, dzs, gamma, grad = ws_case(1, 16, 768, 12, seed=12)
    rb, rd, rg = (rounded(a, F32) for a in (base, dzs, gamma))
    tb, td, tg = dev(base), [dev(d) for d in dzs], dev(gamma)
    out = T.triangular_accumulate_b4_12_ptr_traceable(tb, *td, tg)
    assert_f32(host(out), O.triangular_np(rb, list(rd), rg), what="12 layers")
    for bad in (0, 12):
        with pytest.raises((ValueError, RuntimeError)):
            torch.ops.jit_thc.triangular_accumulate_b4_12_ptr_active(tb, *td, tg, bad)
    with pytest.raises((ValueError, RuntimeError)):
        T.triangular_accumulate_b4_12_ptr_traceable(tb, *td, tg[:11])


# ---------------------------------------------------------------------------
# all_base_b4_12 / all_base_b4_12_split
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dt,B,G,C,L", [(BF16, 2, 16, 768, 12), (F32, 1, 32, 64, 24), (F32, 3, 4, 20, 3)])
def test_all_base_forward_backward(coracle, dt, B, G, C, L):
    print(f"case dt={dt} B={B} G={G} C={C} L={L}", flush=True)
    d = O.make_inputs(B, G, C, L, seed=L, grads=True)
    gen = torch.Generator().manual_seed(100 + L)
    alphas = (torch.randn((L, C, 16), generator=gen) * 0.01 + 1 / 16).numpy()
    x0, gb = d["x0"], d["grad_z"]
    rx, ra, rgb = rounded(x0, dt), rounded(alphas, dt), rounded(gb, dt)

    tx, ta = dev(x0, dt).requires_grad_(), dev(alphas, dt).requires_grad_()
    out = T.all_base_b4_12_traceable(tx, ta)
    assert out.shape == (L, B, G * G, C) and out.dtype == dt
    refs = coracle.Cread_multi(rx, list(ra), G)
    for l in range(L):
        check(host(out[l]), refs[l], dt, f"base[{l}]")
    out.backward(dev(gb, dt))
    check(host(tx.grad), coracle.Cwrite(None, list(rgb), list(ra), h=4 * G), dt, "grad_x0")
    check(host(ta.grad), coracle.Cweight_grad(rx, list(rgb), G), dt, "grad_alpha")

    sx, sa = dev(x0, dt).requires_grad_(), dev(alphas, dt).requires_grad_()
    outs = T.all_base_b4_12_split_traceable(sx, sa)
    assert len(outs) == L and all(torch.equal(o, out[l].detach()) for l, o in enumerate(outs))
    torch.autograd.backward(outs, [dev(g, dt) for g in gb])
    assert torch.equal(sx.grad, tx.grad) and torch.equal(sa.grad, ta.grad)


def test_all_base_split_with_unused_outputs():
    """Outputs that do not reach the loss get zero gradient (local_thc_triton_kernels.py:2655-2663)."""
    d = O.make_inputs(2, 8, 64, 4, seed=9, grads=True)
    alphas = (torch.randn((4, 64, 16), generator=torch.Generator().manual_seed(9)) * 0.01 + 1 / 16).numpy()
    x0, gb = d["x0"], d["grad_z"]
    tx, ta = dev(x0).requires_grad_(), dev(alphas).requires_grad_()
    outs = T.all_base_b4_12_split_traceable(tx, ta)
    loss = (outs[1] * dev(gb[1])).sum() + (outs[3] * dev(gb[3])).sum()
    loss.backward()
    ref_x = O.write_np(gb[1], alphas[1], 32) + O.write_np(gb[3], alphas[3], 32)
    assert_f32(host(tx.grad), ref_x, what="grad_x0")
    assert not ta.grad[0].any() and not ta.grad[2].any()
    assert_f32(host(ta.grad[1]), O.weight_grad_np(x0, gb[1], 8), what="grad_alpha1")
    with pytest.raises(ValueError):
        T.all_base_b4_12_traceable(tx.detach(), dev(np.ones((25, 64, 16), np.float32)))


# ---------------------------------------------------------------------------
# the whole non-shared lazy schedule against the naive high-resolution recurrence
# ---------------------------------------------------------------------------
def _t_read(x, a, g):
    b, h, _, c = x.shape
    s = h // g
    w = a.reshape(c, s, s).permute(1, 2, 0)
    return (x.reshape(b, g, s, g, s, c) * w[None, None, :, None, :, :]).sum((2, 4)).reshape(b, g * g, c)


def _t_write(dz, be, h):
    b, m, c = dz.shape
    g = math.isqrt(m)
    s = h // g
    w = be.reshape(c, s, s).permute(1, 2, 0)
    return (dz.reshape(b, g, g, c)[:, :, None, :, None, :] * w[None, None, :, None, :, :]).reshape(b, h, h, c)


@pytest.mark.parametrize("L", [12, 5])
def test_triangular_schedule_matches_naive_recurrence_fp32(L):
    """x_L and every parameter gradient of the lazy schedule (HIP) equal those of the naive per-layer
    read -> branch -> write_add recurrence (torch, float64, CPU) to fp32 accuracy."""
    print(f"case L={L}", flush=True)
    B, G, C = 2, 8, 64
    gen = torch.Generator().manual_seed(L)
    x0 = torch.randn((B, 4 * G, 4 * G, C), generator=gen)
    alphas = torch.randn((L, C, 16), generator=gen) * 0.05 + 1 / 16
    betas = torch.randn((L, C, 16), generator=gen) * 0.3
    ws = torch.randn((L, C, C), generator=gen) / math.sqrt(C)
    r = torch.randn((B, 4 * G, 4 * G, C), generator=gen)
    # the torch restatement used as the reference agrees with the oracle
    np.testing.assert_allclose(_t_read(x0.double(), alphas[0].double(), G).numpy(), O.read_np(x0.numpy(), alphas[0].numpy(), G), rtol=1e-12, atol=1e-12)

    def run(dev_, dtype, lazy):
        leaves = [t.to(dev_, dtype).requires_grad_() for t in (x0, alphas, betas, ws)]
        tx, ta, tb, tw = leaves

        def branch(l, z):
            return torch.tanh(z @ tw[l]) * 0.5

        if lazy:
            xl = T.triangular_lazy_schedule(tx, ta, tb, branch)
        else:
            x = tx
            for l in range(L):
                x = x + _t_write(branch(l, _t_read(x, ta[l], G)), tb[l], 4 * G)
            xl = x
        (xl * r.to(dev_, dtype)).sum().backward()
        return [xl.detach()] + [t.grad for t in leaves]

    got = run(DEV, F32, True)
    ref = run("cpu", torch.float64, False)
    for name, a, b in zip(("x_L", "grad_x0", "grad_alpha", "grad_beta", "grad_w"), got, ref):
        assert_f32(host(a), b.numpy(), what=name)
