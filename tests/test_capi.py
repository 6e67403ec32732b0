"""C ABI of libtpo_hip.so: loads, exports every symbol include/tpo.h declares,
and rejects bad arguments before touching the GPU (no compute calls here)."""
import ctypes
import os
import re

import pytest

from tests.conftest import REPO

HEADER = os.path.join(REPO, "include", "tpo.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tpo_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib(tpo):
    from torch_point_ops import _native

    L = ctypes.CDLL(_native.HIP_LIB)
    L.tpo_last_error.restype = ctypes.c_char_p
    return L


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("tpo_chamfer_fwd", "tpo_chamfer_bwd", "tpo_chamfer_workspace_size",
                 "tpo_chamfer_pairs_evaluated", "tpo_knn_fwd", "tpo_knn_bwd",
                 "tpo_fps_fwd", "tpo_fps_workspace_size", "tpo_gather_fwd", "tpo_gather_bwd",
                 "tpo_gather_bwd_workspace_size", "tpo_emd_fwd", "tpo_emd_bwd",
                 "tpo_emd_workspace_size", "tpo_last_error", "tpo_abi_version"):
        assert must in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.tpo_abi_version() >> 16 == 2


def test_argument_errors_are_reported(lib):
    P, I = ctypes.c_void_p, ctypes.c_int64
    lib.tpo_knn_fwd.argtypes = [ctypes.c_int, P, P, P, P, I, I, I, I, I, ctypes.c_int,
                                ctypes.c_int, P, P, P, P, I, P]
    rc = lib.tpo_knn_fwd(0, None, None, None, None, 1, 4, 4, 3, 2, 3, -1, None, None, None, None,
                         0, None)
    assert rc == -1 and b"Norm must be 1 or 2" in lib.tpo_last_error()
    lib.tpo_fps_fwd.argtypes = [ctypes.c_int, P, I, I, I, P, P, I, P]
    assert lib.tpo_fps_fwd(0, None, 2, 10, 11, None, None, 0, None) == -1
    assert b"nsamples" in lib.tpo_last_error()
    lib.tpo_fps_workspace_size.argtypes = [ctypes.c_int, I, I]
    lib.tpo_fps_workspace_size.restype = I
    ws = lib.tpo_fps_workspace_size(0, 16, 65536)
    assert ws >= 16 * 65536 * 20 and ws % 256 == 0
    assert lib.tpo_fps_fwd(0, None, 2, 10, 5, None, None, 0, None) == -4  # no workspace
    assert lib.tpo_fps_workspace_size(9, 1, 10) == -1
    lib.tpo_chamfer_fwd.argtypes = [ctypes.c_int, P, P, I, I, I, P, P, P, P, P, I, P]
    assert lib.tpo_chamfer_fwd(0, None, None, -1, 3, 3, None, None, None, None, None, 0,
                               None) == -1
    assert lib.tpo_chamfer_fwd(7, None, None, 0, 3, 3, None, None, None, None, None, 0,
                               None) == 0  # B=0
    lib.tpo_chamfer_workspace_size.argtypes = [ctypes.c_int, I, I, I]
    lib.tpo_chamfer_workspace_size.restype = I
    assert lib.tpo_chamfer_workspace_size(0, 32, 8192, 8192) > 32 * 16384 * 20
    assert lib.tpo_chamfer_workspace_size(0, 2, 100, 8192) == 0    # too small to prune
    assert lib.tpo_chamfer_workspace_size(1, 32, 8192, 8192) == 0  # no pruned double path
    assert lib.tpo_chamfer_workspace_size(2, 32, 8192, 8192) == \
        lib.tpo_chamfer_workspace_size(0, 32, 8192, 8192)  # half: same float4 layout
    assert lib.tpo_chamfer_workspace_size(0, -1, 3, 3) == -1
    # fused module loss: the forward's workspace (grid search or none), both
    # distance arrays, 2 x 256 chunk sums (doubles), a workgroup counter;
    # 256-byte regions
    lib.tpo_chamfer_loss_workspace_size.argtypes = [ctypes.c_int, I, I, I]
    lib.tpo_chamfer_loss_workspace_size.restype = I
    assert lib.tpo_chamfer_loss_workspace_size(0, 32, 8192, 8192) == \
        lib.tpo_chamfer_workspace_size(0, 32, 8192, 8192) + 2 * 32 * 8192 * 4 + 4096 + 256
    # double: dist1 1600 -> 1792 bytes (256-byte regions), dist2 1024, chunk sums 4096
    assert lib.tpo_chamfer_loss_workspace_size(1, 2, 100, 64) == 1792 + 1024 + 4096 + 256
    assert lib.tpo_chamfer_loss_workspace_size(9, 2, 100, 64) == -1
    lib.tpo_chamfer_loss_fwd.argtypes = [ctypes.c_int, P, P, I, I, I, ctypes.c_int, P, P, P, P,
                                         I, P]
    fake = ctypes.c_void_p(4096)  # never dereferenced: the calls fail their checks first
    assert lib.tpo_chamfer_loss_fwd(0, fake, fake, 2, 8, 8, 1, None, fake, fake, fake, 1 << 20,
                                    None) == -1  # no loss output
    assert lib.tpo_chamfer_loss_fwd(0, fake, fake, 2, 8, 8, 1, fake, fake, fake, None, 0,
                                    None) == -4  # no workspace
    assert b"workspace" in lib.tpo_last_error()
    assert lib.tpo_chamfer_loss_fwd(5, fake, fake, 2, 8, 8, 1, fake, fake, fake, fake, 1 << 20,
                                    None) == -2  # dtype
    lib.tpo_chamfer_pairs_evaluated.argtypes = [ctypes.c_int, P, I, I, I, P, P]
    assert lib.tpo_chamfer_pairs_evaluated(0, None, 2, 4096, 4096, None, None) == -1
    lib.tpo_knn_workspace_size.argtypes = [ctypes.c_int, I, I, I, I, I, ctypes.c_int]
    lib.tpo_knn_workspace_size.restype = I
    # float 3-D against long clouds: the query order, then the reference grid
    # (8 floats of box per cloud, 16^3 + 1 cell starts, the indices by cell)
    up = lambda x: (x + 255) // 256 * 256
    assert lib.tpo_knn_workspace_size(0, 8, 16384, 16384, 3, 16, 2) == \
        8 * 16384 * 4 + up(8 * 8 * 4) + up(8 * 4097 * 4) + up(8 * 16384 * 4)
    assert lib.tpo_knn_workspace_size(1, 8, 16384, 16384, 3, 16, 2) == 8 * 16384 * 4  # order only
    assert lib.tpo_knn_workspace_size(0, 8, 16384, 1000, 3, 16, 2) == 8 * 16384 * 4  # short clouds
    # bf16: squared norms (float per point), a partial list of K (distance,
    # index) keys per query and reference slice of the exact pass (config 5:
    # 8 slices), then for clouds of >= 4096 references the sampled bound's
    # 8 x 8 floats per query, the rerun counts (int32 per cloud) and lists
    # (int32 per query), and per query and slice of the candidate pass
    # (config 5: 12 slices) 128 candidate keys and two int32 counts
    assert lib.tpo_knn_workspace_size(3, 4, 4096, 65536, 128, 32, 2) == \
        4 * (4096 + 65536) * 4 + 4 * 4096 * 8 * 32 * 8 + 4 * 4096 * 64 * 4 + 256 + \
        4 * 4096 * 4 + 4 * 4096 * 12 * 128 * 8 + 4 * 4096 * 12 * 2 * 4
    assert lib.tpo_knn_workspace_size(3, 2, 100, 1000, 64, 8, 2) == \
        up(2 * (128 + 1024) * 4) + up(2 * 100 * 2 * 8 * 8)  # 2 slices; short clouds: no bound
    assert lib.tpo_knn_workspace_size(3, 4, 4096, 65536, 128, 32, 1) == 0  # no bf16 L1 kernel
    assert lib.tpo_knn_workspace_size(3, 4, 4096, 65536, 130, 32, 2) == 0  # D % 8 != 0
    assert lib.tpo_knn_fwd(3, None, None, None, None, 1, 4, 4, 3, 2, 2, -1, None, None, None,
                           None, 0, None) == -2  # bf16 with D=3: unsupported
    lib.tpo_gather_bwd_workspace_size.argtypes = [I, I]
    lib.tpo_gather_bwd_workspace_size.restype = I
    assert lib.tpo_gather_bwd_workspace_size(16, 65536) == 16 * 65536 * 4


def test_emd_sizes_and_errors(lib):
    P, I = ctypes.c_void_p, ctypes.c_int64
    lib.tpo_emd_workspace_size.argtypes = [ctypes.c_int, I, I, I]
    lib.tpo_emd_workspace_size.restype = I
    # float/half: p1, p2 (4 floats a point), remain, 10 levels of ratios,
    # 8 x 64 cost partials, 16 row tiles of grad_xyz1 partials and 8 column
    # tiles of grad_xyz2 partials per cloud, plus the int32 point orders
    B, n, m = 16, 2048, 2048
    vals = B * (n * 4 + m * 4 + n + m + 10 * n + 10 * m + 8 * 64 + 16 * n * 3 + 8 * m * 3)
    assert lib.tpo_emd_workspace_size(0, B, n, m) == 4 * vals + 4 * B * (n + m)
    assert lib.tpo_emd_workspace_size(2, B, n, m) == 4 * vals + 4 * B * (n + m)
    assert lib.tpo_emd_workspace_size(1, B, n, m) == 8 * vals + 4 * B * (n + m)
    assert lib.tpo_emd_workspace_size(0, 2, 0, 5) == 0
    assert lib.tpo_emd_workspace_size(3, 1, 4, 4) == -1  # bfloat16: not an EMD dtype
    lib.tpo_emd_fwd.argtypes = [ctypes.c_int, P, P, I, I, I, P, P, P, I, P]
    assert lib.tpo_emd_fwd(0, None, None, 1, -1, 4, None, None, None, 0, None) == -1
    assert b"bad sizes" in lib.tpo_last_error()
    assert lib.tpo_emd_fwd(3, None, None, 1, 4, 4, None, None, None, 0, None) == -2
    assert lib.tpo_emd_fwd(0, None, None, 1, 4, 4, None, None, None, 0, None) == -4
    assert b"workspace" in lib.tpo_last_error()
    lib.tpo_emd_bwd.argtypes = [ctypes.c_int, P, P, P, P, I, I, I, P, P, P, I, P]
    assert lib.tpo_emd_bwd(0, None, None, None, None, 1, 4, 4, None, None, None, 0, None) == -4
    assert lib.tpo_emd_bwd(0, None, None, None, None, 1 << 31, 4, 4, None, None, None, 0,
                           None) == -1
