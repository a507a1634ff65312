"""GPU parity of the legacy per-block functions and modules (MI355X only).

``ops.local_write / local_read / local_read_add`` and their ``_no_weight_grad`` forms
(local_thc_triton_kernels.py:1379-1575) and the ``ChannelwiseLocalTokenHyperConnectionTriton*``
modules (local_thc.py:511-617), against the CPU oracle's read / write / weight-gradient
(pinned in tests/test_oracle.py).  Tolerances as in test_gpu_parity.
"""

from __future__ import annotations

import pytest
import torch

from flowmatching_lthc_amd import local_thc as LT
from flowmatching_lthc_amd import ops
from oracle import oracle as O

from .test_gpu_parity import BF16, F32, assert_bf16, assert_f32, dev, host, rounded

pytestmark = pytest.mark.gpu


def case(B=2, G=16, C=256, seed=0):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn((B, 4 * G, 4 * G, C), generator=gen).numpy()
    z = (torch.randn((B, G * G, C), generator=gen) * 0.5).numpy()
    w = (torch.randn((C, 16), generator=gen) * 0.1 + 1 / 16).numpy()
    gx = (torch.randn((B, 4 * G, 4 * G, C), generator=gen) * 1e-2).numpy()
    gz = (torch.randn((B, G * G, C), generator=gen) * 1e-2).numpy()
    return x, z, w, gx, gz


def check(got, ref, dtype, what):
    (assert_f32 if dtype == F32 else assert_bf16)(got, ref, what=what)


@pytest.mark.parametrize("dt", [F32, BF16])
def test_legacy_functions_forward_backward(dt):
    print(f"case dt={dt}", flush=True)
    x, z, w, gx, gz = case(seed=1)
    rx, rz, rw, rgx, rgz = (rounded(a, dt) for a in (x, z, w, gx, gz))
    G = 16

    # read (legacy name local_write) and its frozen form
    tx, tw = dev(x, dt).requires_grad_(), dev(w, dt).requires_grad_()
    out = ops.local_write(tx, tw)
    check(host(out), O.read_np(rx, rw, G), dt, "local_write")
    out.backward(dev(gz, dt))
    check(host(tx.grad), O.write_np(rgz, rw, 4 * G), dt, "local_write dX")
    check(host(tw.grad), O.weight_grad_np(rx, rgz, G), dt, "local_write dW")
    fx, fw = dev(x, dt).requires_grad_(), dev(w, dt).requires_grad_()
    out_f = ops.local_write_no_weight_grad(fx, fw)
    assert torch.equal(out_f, out.detach())
    out_f.backward(dev(gz, dt))
    assert torch.equal(fx.grad, tx.grad) and fw.grad is None

    # write (legacy name local_read)
    tz, tw = dev(z, dt).requires_grad_(), dev(w, dt).requires_grad_()
    out = ops.local_read(tz, tw)
    check(host(out), O.write_np(rz, rw, 4 * G), dt, "local_read")
    out.backward(dev(gx, dt))
    check(host(tz.grad), O.read_np(rgx, rw, G), dt, "local_read dZ")
    check(host(tw.grad), O.weight_grad_np(rgx, rz, G), dt, "local_read dW")

    # fused write + residual add and its frozen form
    tz, tw, tx = dev(z, dt).requires_grad_(), dev(w, dt).requires_grad_(), dev(x, dt).requires_grad_()
    out = ops.local_read_add(tz, tw, tx)
    check(host(out), O.write_add_np(rx, rz, rw), dt, "local_read_add")
    out.backward(dev(gx, dt))
    assert torch.equal(tx.grad, dev(gx, dt))
    check(host(tz.grad), O.read_np(rgx, rw, G), dt, "local_read_add dZ")
    check(host(tw.grad), O.weight_grad_np(rgx, rz, G), dt, "local_read_add dW")
    fz, fw, fx = dev(z, dt).requires_grad_(), dev(w, dt).requires_grad_(), dev(x, dt).requires_grad_()
    out_f = ops.local_read_add_no_weight_grad(fz, fw, fx)
    assert torch.equal(out_f, out.detach())
    out_f.backward(dev(gx, dt))
    assert torch.equal(fz.grad, tz.grad) and torch.equal(fx.grad, tx.grad) and fw.grad is None


def test_hyper_connection_modules():
    B, G, C = 2, 16, 128
    x, z, _, gx, _ = case(B, G, C, seed=2)
    mods = {
        "plain": LT.ChannelwiseLocalTokenHyperConnectionTriton(4 * G, G, C, C),
        "read_add": LT.ChannelwiseLocalTokenHyperConnectionTritonReadAdd(4 * G, G, C, C),
        "frozen": LT.ChannelwiseLocalTokenHyperConnectionTritonFrozen(4 * G, G, C, C),
        "traceable": LT.ChannelwiseLocalTokenHyperConnectionTritonTraceable(4 * G, G, C, C),
    }
    gen = torch.Generator().manual_seed(3)
    logits = torch.randn((C, 16), generator=gen)
    wgt = torch.randn((C, 16), generator=gen) * 0.3 + 1.0
    for m in mods.values():
        with torch.no_grad():
            m.read_logits.copy_(logits)
            m.write_weight.copy_(wgt)
        m.cuda()
    alpha = torch.softmax(logits.double(), -1).numpy()
    ref_read = O.read_np(x, alpha, G)
    ref_write_add = O.write_add_np(x, z, wgt.numpy())
    for name, m in mods.items():
        tx = dev(x).requires_grad_()
        zz = m.read(tx)
        assert_f32(host(zz), ref_read, what=f"{name} read")
        tz = dev(z).requires_grad_()
        if name == "plain":
            out = tx + m.write(tz)
        else:
            out = m.write_add(tz, tx)
        assert_f32(host(out), ref_write_add, what=f"{name} write_add")
        (zz.sum() + (out * dev(gx)).sum()).backward()
        frozen = name == "frozen"
        assert (m.read_logits.grad is None) == frozen and (m.write_weight.grad is None) == frozen, name
        if not frozen:
            assert_f32(host(m.write_weight.grad), O.weight_grad_np(gx, z, G), what=f"{name} dW")
    for name in ("frozen", "traceable"):
        with pytest.raises(NotImplementedError):
            mods[name].write(dev(z))
