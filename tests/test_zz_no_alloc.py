"""tpo_chamfer_fwd_noalloc (the allocation-free Chamfer forward) against
tpo_chamfer_fwd with a caller-provided workspace, through the C ABI: bit for
bit, on two calls in a row (the second smaller, so the static scratch holds
the first call's contents), for the grid-search and dense paths, and the
rejection of sizes beyond the static scratch."""
import ctypes

import pytest
import torch

import workloads

P, I = ctypes.c_void_p, ctypes.c_int64


@pytest.fixture(scope="module")
def lib(tpo):
    from torch_point_ops import _native

    L = ctypes.CDLL(_native.HIP_LIB)
    L.tpo_last_error.restype = ctypes.c_char_p
    L.tpo_chamfer_fwd.argtypes = [ctypes.c_int, P, P, I, I, I, P, P, P, P, P, I, P]
    L.tpo_chamfer_fwd_noalloc.argtypes = [ctypes.c_int, P, P, I, I, I, P, P, P, P, P]
    L.tpo_chamfer_workspace_size.argtypes = [ctypes.c_int, I, I, I]
    L.tpo_chamfer_workspace_size.restype = I
    L.tpo_chamfer_noalloc_max_workspace.restype = I
    return L


def _outs(B, N, M, dtype, dev):
    return (torch.full((B, N), -7.0, device=dev, dtype=dtype),
            torch.full((B, M), -7.0, device=dev, dtype=dtype),
            torch.full((B, N), -7, dtype=torch.int32, device=dev),
            torch.full((B, M), -7, dtype=torch.int32, device=dev))


def _run(lib, fn, code, p1, p2, dev, ws=None):
    B, N, M = p1.shape[0], p1.shape[1], p2.shape[1]
    d1, d2, i1, i2 = _outs(B, N, M, p1.dtype, dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [code, p1.data_ptr(), p2.data_ptr(), B, N, M, d1.data_ptr(), d2.data_ptr(),
            i1.data_ptr(), i2.data_ptr()]
    if fn == "noalloc":
        rc = lib.tpo_chamfer_fwd_noalloc(*args, stream)
    else:
        rc = lib.tpo_chamfer_fwd(*args, None if ws is None else ws.data_ptr(),
                                 0 if ws is None else ws.numel(), stream)
    assert rc == 0, lib.tpo_last_error()
    torch.cuda.synchronize()
    return d1, d2, i1, i2


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_noalloc_matches_workspace_entry_point(tpo, lib, dev, dtype):
    code = 0 if dtype == torch.float32 else 2
    big = [t.to(dev, dtype) for t in workloads.chamfer_c2(seed=3)]          # B=32, N=M=8192
    g = torch.Generator().manual_seed(4)
    small = [(torch.rand(3, 3000, 3, generator=g)).to(dev, dtype),
             (torch.rand(3, 2500, 3, generator=g)).to(dev, dtype)]          # grid path, smaller
    tiny = [(torch.rand(2, 300, 3, generator=g)).to(dev, dtype),
            (torch.rand(2, 257, 3, generator=g)).to(dev, dtype)]            # dense path
    for p1, p2 in (big, small, tiny):
        B, N, M = p1.shape[0], p1.shape[1], p2.shape[1]
        print(f"noalloc case dtype={dtype} B={B} N={N} M={M}", flush=True)
        need = lib.tpo_chamfer_workspace_size(code, B, N, M)
        assert need <= lib.tpo_chamfer_noalloc_max_workspace()
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev) if need > 0 else None
        want = _run(lib, "ws", code, p1, p2, dev, ws)
        got = _run(lib, "noalloc", code, p1, p2, dev)
        for a, b in zip(got, want):
            assert torch.equal(a, b)


@pytest.mark.gpu
def test_noalloc_rejects_sizes_beyond_scratch(tpo, lib, dev):
    # B=64, N=M=16384 needs ~77 MB of workspace: refused before any launch
    B, N, M = 64, 16384, 16384
    assert lib.tpo_chamfer_workspace_size(0, B, N, M) > lib.tpo_chamfer_noalloc_max_workspace()
    rc = lib.tpo_chamfer_fwd_noalloc(0, None, None, B, N, M, None, None, None, None, None)
    assert rc == -4
    assert b"static scratch" in lib.tpo_last_error()
