"""lthc_materialise_bwd_noalloc (the materialise backward with its partial sums in the library's per-GPU scratch
array, for callers that cannot allocate) against lthc_materialise_bwd with a caller workspace: the same kernels and
launch plan, so gdZ and gbeta are bitwise equal.  Two calls in a row, the second with a smaller input (the scratch
array keeps the first call's partials; the second must not read them), then the first shape again; a shape whose
partials exceed the scratch array is refused before anything is launched.  Collected last (test_zz_*), so a failure
here hides no other test."""

import ctypes

import pytest
import torch

from flowmatching_lthc_amd import _abi

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(B, G, C, L, dtype, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    H = 4 * G
    g = (torch.randn((B, H, H, C), generator=gen, device=DEV) * 1e-3).to(dtype)
    dzs = [(torch.randn((B, G * G, C), generator=gen, device=DEV) * 0.02).to(dtype) for _ in range(L)]
    betas = [torch.randn((C, 16), generator=gen, device=DEV) * 0.02 for _ in range(L)]
    return g, dzs, betas


def _with_workspace(lib, g, dzs, betas, B, G, C, L):
    gdz = [torch.empty_like(z) for z in dzs]
    gb = torch.empty((L, C, 16), device=DEV)
    ws = torch.empty((int(lib.lthc_materialise_bwd_workspace_bytes(B, G, 4, C, L)) + 16,), device=DEV, dtype=torch.uint8)
    rc = lib.lthc_materialise_bwd(
        g.data_ptr(), _abi.code(g), _abi.ptr_array(dzs), _abi.ptr_array(betas), _abi.F32, _abi.ptr_array(gdz),
        gb.data_ptr(), B, G, 4, C, L, ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream,
    )  # fmt: skip
    _abi.check(rc, "lthc_materialise_bwd")
    return gdz, gb


def _noalloc(lib, g, dzs, betas, B, G, C, L):
    gdz = [torch.empty_like(z) for z in dzs]
    gb = torch.empty((L, C, 16), device=DEV)
    rc = lib.lthc_materialise_bwd_noalloc(
        g.data_ptr(), _abi.code(g), _abi.ptr_array(dzs), _abi.ptr_array(betas), _abi.F32, _abi.ptr_array(gdz),
        gb.data_ptr(), B, G, 4, C, L, torch.cuda.current_stream().cuda_stream,
    )  # fmt: skip
    _abi.check(rc, "lthc_materialise_bwd_noalloc")
    return gdz, gb


def test_materialise_bwd_noalloc_equals_workspace_entry():
    lib = _abi.load()
    assert lib.lthc_noalloc_scratch_bytes() == 64 << 20
    shapes = [
        (64, 16, 768, 12, torch.bfloat16),  # configuration 3 (the tile kernel)
        (2, 8, 128, 5, torch.float16),  # smaller, another depth bucket
        (3, 4, 64, 2, torch.float32),  # fp32: the older single-pass kernel
        (64, 16, 768, 12, torch.bfloat16),  # the first shape again after the smaller calls
    ]
    for i, (B, G, C, L, dt) in enumerate(shapes):
        print(f"case noalloc B={B} G={G} C={C} L={L} {dt}", flush=True)
        assert lib.lthc_materialise_bwd_workspace_bytes(B, G, 4, C, L) <= lib.lthc_noalloc_scratch_bytes()
        g, dzs, betas = _inputs(B, G, C, L, dt, seed=40 + i)
        ref_dz, ref_gb = _with_workspace(lib, g, dzs, betas, B, G, C, L)
        got_dz, got_gb = _noalloc(lib, g, dzs, betas, B, G, C, L)
        torch.cuda.synchronize()
        for l in range(L):
            assert torch.equal(got_dz[l], ref_dz[l]), f"gdZ_{l}"
        assert torch.equal(got_gb, ref_gb), "gbeta"


def test_materialise_bwd_noalloc_refuses_shapes_beyond_the_scratch_array():
    lib = _abi.load()
    B, G, L = 1, 16, 48
    for C in (8192, 16384, 65536):  # the first width whose partials exceed the scratch array
        need = int(lib.lthc_materialise_bwd_workspace_bytes(B, G, 4, C, L))
        if need > lib.lthc_noalloc_scratch_bytes():
            break
    assert need > lib.lthc_noalloc_scratch_bytes()
    fake = ctypes.c_void_p(4096)  # never dereferenced: the size check comes first
    arr = (ctypes.c_void_p * L)(*([4096] * L))
    rc = lib.lthc_materialise_bwd_noalloc(fake, _abi.BF16, arr, arr, _abi.F32, arr, fake, B, G, 4, C, L, None)
    assert rc == _abi.ERR_UNSUPPORTED
    assert "scratch" in lib.lthc_last_error().decode()
