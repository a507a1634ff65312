"""lthc_materialise_bwd_noalloc (the materialise backward with its partial sums in the library's per-GPU scratch
array, for callers that cannot allocate) against lthc_materialise_bwd with a caller workspace: the same kernels and
launch plan, so gdZ and gbeta are bitwise equal.  Two calls in a row, the second with a smaller input (the scratch
array keeps the first call's partials; the second must not read them), then the first shape again; a call captured in
a HIP graph and replayed; a shape whose partials exceed the scratch array is refused before anything is launched.
Collected last (test_zz_*), so a failure here hides no other test."""

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
        (4, 16, 256, 20, torch.bfloat16),  # the depth-24 bucket (8 wavefronts, two column blocks of layers)
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
    """Every pointer is a real device tensor of the shape it names, so a launch before the size check could only
    change the result, never touch memory that is not there."""
    lib = _abi.load()
    B, G, L = 1, 16, 48
    for C in (8192, 16384, 65536):  # the first width whose partials exceed the scratch array
        need = int(lib.lthc_materialise_bwd_workspace_bytes(B, G, 4, C, L))
        if need > lib.lthc_noalloc_scratch_bytes():
            break
    assert need > lib.lthc_noalloc_scratch_bytes()
    print(f"case noalloc refusal B={B} G={G} C={C} L={L}", flush=True)
    g, dzs, betas = _inputs(B, G, C, L, torch.bfloat16, seed=7)
    gdz = [torch.empty_like(z) for z in dzs]
    gb = torch.empty((L, C, 16), device=DEV)
    rc = lib.lthc_materialise_bwd_noalloc(
        g.data_ptr(), _abi.BF16, _abi.ptr_array(dzs), _abi.ptr_array(betas), _abi.F32, _abi.ptr_array(gdz),
        gb.data_ptr(), B, G, 4, C, L, torch.cuda.current_stream().cuda_stream,
    )  # fmt: skip
    assert rc == _abi.ERR_UNSUPPORTED
    assert "scratch" in lib.lthc_last_error().decode()
    torch.cuda.synchronize()


def test_materialise_bwd_noalloc_under_graph_capture():
    """The entry point inside a captured HIP graph (torch.cuda.graph): one eager call first (the per-device scratch
    address and the occupancy queries are looked up on first use, outside capture), then the call captured and the
    graph replayed three times with eager work and synchronisations between the replays; every replay equals
    lthc_materialise_bwd with a caller workspace bit for bit, on inputs refilled between replays."""
    lib = _abi.load()
    B, G, C, L = 8, 16, 768, 12
    print(f"case noalloc graph B={B} G={G} C={C} L={L}", flush=True)
    g, dzs, betas = _inputs(B, G, C, L, torch.bfloat16, seed=90)
    _noalloc(lib, g, dzs, betas, B, G, C, L)  # first call on the device: eager
    torch.cuda.synchronize()
    gdz = [torch.empty_like(z) for z in dzs]
    gb = torch.empty((L, C, 16), device=DEV)
    dz_ptrs, beta_ptrs, out_ptrs = _abi.ptr_array(dzs), _abi.ptr_array(betas), _abi.ptr_array(gdz)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = lib.lthc_materialise_bwd_noalloc(
                g.data_ptr(), _abi.BF16, dz_ptrs, beta_ptrs, _abi.F32, out_ptrs, gb.data_ptr(), B, G, 4, C, L,
                side.cuda_stream,
            )  # fmt: skip
    torch.cuda.current_stream().wait_stream(side)
    _abi.check(rc, "lthc_materialise_bwd_noalloc (captured)")
    gen = torch.Generator(device=DEV).manual_seed(91)
    for rep in range(3):
        g.copy_((torch.randn(g.shape, generator=gen, device=DEV) * 1e-3).to(g.dtype))
        for z in dzs:
            z.copy_((torch.randn(z.shape, generator=gen, device=DEV) * 0.02).to(z.dtype))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref_dz, ref_gb = _with_workspace(lib, g, dzs, betas, B, G, C, L)
        torch.cuda.synchronize()
        for l in range(L):
            assert torch.equal(gdz[l], ref_dz[l]), f"replay {rep}: gdZ_{l}"
        assert torch.equal(gb, ref_gb), f"replay {rep}: gbeta"
