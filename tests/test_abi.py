"""C ABI and host-side logic — CPU only (no kernel is launched here)."""

import ctypes
import os
import re

import pytest
import torch

from flowmatching_lthc_amd import _abi, ops
from flowmatching_lthc_amd.local_thc import LayerLocalWrite, SharedLocalRead

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lthc.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lthc_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _abi.load()
    names = declared_functions()
    assert len(names) >= 11
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(_abi.EXPORTS) == names
    assert lib.lthc_abi_version() == 3


def _err(rc):
    return rc, _abi.load().lthc_last_error().decode()


def test_argument_errors_are_reported_without_launching():
    lib = _abi.load()
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    rc, msg = _err(lib.lthc_read_fwd(fake, _abi.BF16, fake, _abi.F32, fake, 2, 16, 3, 768, None))
    assert rc == _abi.ERR_UNSUPPORTED and "s == 4" in msg
    rc, msg = _err(lib.lthc_read_fwd(fake, _abi.BF16, fake, _abi.F32, fake, 2, 16, 4, 770, None))
    assert rc == _abi.ERR_INVALID and "multiple of 4" in msg
    rc, msg = _err(lib.lthc_read_fwd(fake, 7, fake, _abi.F32, fake, 2, 16, 4, 768, None))
    assert rc == _abi.ERR_INVALID and "dtype" in msg
    rc, msg = _err(lib.lthc_read_fwd(None, _abi.BF16, fake, _abi.F32, fake, 2, 16, 4, 768, None))
    assert rc == _abi.ERR_INVALID and "x is NULL" in msg
    arr = (ctypes.c_void_p * 1)(4096)
    rc, msg = _err(lib.lthc_materialise_fwd(None, arr, _abi.BF16, arr, _abi.F32, fake, 2, 16, 4, 768, 0, None))
    assert rc == _abi.ERR_INVALID and "L must be" in msg
    rc, msg = _err(lib.lthc_materialise_fwd(None, arr, _abi.BF16, arr, _abi.F32, fake, 2, 16, 4, 768, 49, None))
    assert rc == _abi.ERR_UNSUPPORTED
    rc, msg = _err(lib.lthc_recur_fwd(fake, fake, _abi.F32, fake, _abi.F32, fake, 10, 6, None))
    assert rc == _abi.ERR_INVALID
    misaligned = ctypes.c_void_p(4096 + 2)
    rc, msg = _err(lib.lthc_read_fwd(misaligned, _abi.BF16, fake, _abi.F32, fake, 2, 16, 4, 768, None))
    assert rc == _abi.ERR_INVALID and "aligned" in msg
    rc, msg = _err(lib.lthc_weight_grad(fake, arr, _abi.F32, fake, 2, 16, 4, 768, 1, None, 0, None))
    assert rc == _abi.ERR_INVALID and "workspace" in msg
    rc, msg = _err(lib.lthc_qk_norm_rope(fake, _abi.BF16, fake, fake, _abi.F32, fake, fake, _abi.F32, fake, fake, 2, 256, 12, 32, 1e-6, None))
    assert rc == _abi.ERR_UNSUPPORTED and "64" in msg
    rc, msg = _err(lib.lthc_qk_norm_rope(fake, _abi.BF16, None, fake, _abi.F32, fake, fake, _abi.F32, fake, fake, 2, 256, 12, 64, 1e-6, None))
    assert rc == _abi.ERR_INVALID and "NULL" in msg
    rc, msg = _err(lib.lthc_norm_modulate_fwd(fake, _abi.BF16, fake, _abi.F32, fake, fake, 766, fake, None, 2, 256, 768, 1e-6, None))
    assert rc == _abi.ERR_INVALID and "mod_ld" in msg
    rc, msg = _err(lib.lthc_gate_residual(fake, fake, 772, fake, _abi.BF16, fake, 2, 256, 768, None))
    assert rc == _abi.ERR_INVALID and "gate_ld" in msg
    rc, msg = _err(lib.lthc_swiglu(fake, _abi.BF16, fake, 16, 12, None))
    assert rc == _abi.ERR_UNSUPPORTED and "multiple of 8" in msg
    rc, msg = _err(lib.lthc_swiglu(ctypes.c_void_p(4096 + 8), _abi.BF16, fake, 16, 16, None))
    assert rc == _abi.ERR_INVALID and "aligned" in msg

    # the whole-interface entry points: NULL arrays, a missing workspace (before any launch)
    arrs = (ctypes.c_void_p * 12)(*([4096] * 12))
    rc, msg = _err(lib.lthc_interface_bwd(fake, None, _abi.BF16, fake, arrs, fake, arrs, _abi.F32, fake, arrs, fake,
                                          fake, 2, 16, 4, 768, 12, None, 0, None))  # fmt: skip
    assert rc == _abi.ERR_INVALID and "NULL" in msg
    rc, msg = _err(lib.lthc_interface_bwd(fake, arrs, _abi.BF16, fake, arrs, fake, arrs, _abi.F32, fake, arrs, fake,
                                          fake, 2, 16, 4, 768, 12, None, 0, None))  # fmt: skip
    assert rc == _abi.ERR_INVALID and "workspace" in msg
    rc, msg = _err(lib.lthc_interface_fwd(fake, _abi.BF16, fake, arrs, _abi.F32, arrs, None, fake, 2, 16, 4, 768, 12,
                                          None, 0, None))  # fmt: skip
    assert rc == _abi.ERR_INVALID and "z (L + 1 outputs)" in msg
    assert _abi.load().lthc_interface_workspace_bytes(2, 16, 4, 768, 0) == 0


def test_workspace_sizes_are_consistent():
    n = _abi.weight_grad_workspace_bytes(256, 16, 4, 768, 12)
    assert n > 0 and n % (12 * 768 * 16 * 4) == 0
    assert _abi.weight_grad_workspace_bytes(0, 16, 4, 768, 12) == 0
    # one partial row of C floats per block row; block rows = min(8-row chunks (4 row lanes x 2 rows), 256)
    assert _abi.recur_bwd_workspace_bytes(65536, 768) == 256 * 768 * 4
    assert _abi.recur_bwd_workspace_bytes(100, 768) == 13 * 768 * 4


def test_ops_refuse_cpu_tensors():
    x = torch.randn(1, 64, 64, 8)
    w = torch.full((8, 16), 1 / 16)
    with pytest.raises(ValueError, match="no CPU fallback"):
        ops.local_write_traceable(x, w)
    with pytest.raises(ValueError, match="no CPU fallback"):
        ops.final_accumulate_b4_traceable(x, torch.zeros(2, 1, 256, 8), torch.ones(2, 8, 16))
    from flowmatching_lthc_amd import ops_branch

    with pytest.raises(ValueError, match="no CPU fallback"):
        ops_branch.swiglu(torch.zeros(4, 32))
    with pytest.raises(ValueError, match="no CPU fallback"):
        ops_branch.qk_norm_rope(torch.zeros(1, 4, 3, 2, 64), torch.ones(64), torch.ones(64), torch.ones(4, 64), torch.zeros(4, 64), 1e-6)


def test_fake_shapes_propagate_on_meta():
    x = torch.empty(2, 64, 64, 768, device="meta", dtype=torch.bfloat16)
    w = torch.empty(768, 16, device="meta")
    z = torch.ops.jit_thc.local_write_traceable(x, w)
    assert z.shape == (2, 256, 768) and z.dtype == torch.bfloat16
    xx = torch.ops.jit_thc.local_read_traceable(z, w)
    assert xx.shape == x.shape
    dzs = [torch.empty(2, 256, 768, device="meta", dtype=torch.bfloat16) for _ in range(12)]
    bs = [torch.empty(768, 16, device="meta") for _ in range(12)]
    out = torch.ops.jit_thc.final_accumulate_b4_12_traceable(x, *dzs, *bs)
    assert out.shape == x.shape and out.dtype == x.dtype
    gdz = torch.ops.jit_thc.final_accumulate_b4_12_grad_dz_ptr(x, *bs)
    assert gdz.shape == (12, 2, 256, 768)
    gb = torch.ops.jit_thc.final_accumulate_b4_12_grad_beta_ptr(x, *dzs)
    assert gb.shape == (12, 768, 16) and gb.dtype == torch.float32
    zn = torch.ops.jit_thc.lazy_workspace_update(z, z, torch.empty(768, device="meta", dtype=torch.bfloat16))
    assert zn.shape == z.shape


def test_module_shapes_and_names_match_reference():
    r = SharedLocalRead(64, 16, 768, 768)
    w = LayerLocalWrite(64, 16, 768, 768)
    assert set(dict(r.named_parameters())) == {"read_logits"}
    assert set(dict(w.named_parameters())) == {"write_weight"}
    assert r.read_logits.shape == (768, 16) and float(r.read_logits.abs().max()) == 0.0
    assert w.write_weight.shape == (768, 16) and float(w.write_weight.min()) == 1.0
    torch.testing.assert_close(r.alpha(), torch.full((768, 16), 1 / 16))
    with pytest.raises(ValueError, match="divisible"):
        SharedLocalRead(64, 12, 768, 768)
    with pytest.raises(ValueError, match="expected"):
        r.read(torch.empty(1, 32, 32, 768))
    # gamma_from_alpha keeps the reference's dtype semantics
    g = w.gamma_from_alpha(r.alpha(dtype=torch.bfloat16))
    assert g.dtype == torch.bfloat16 and g.shape == (768,)


def test_group_weights_expand_to_channels():
    w = LayerLocalWrite(64, 16, 8, 2)
    w.write_weight.data = torch.arange(32, dtype=torch.float32).reshape(2, 16)
    cb = w.channel_beta()
    assert cb.shape == (8, 16)
    torch.testing.assert_close(cb[3], w.write_weight[0])
    torch.testing.assert_close(cb[4], w.write_weight[1])
