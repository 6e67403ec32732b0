"""numpy front end of the CPU oracle (libtpo_oracle.so).

TEST INFRASTRUCTURE ONLY: the checker used by tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg.  The product package never imports this.

Every function takes and returns numpy arrays.  float16 arrays are passed as
their binary16 bits; the C side does the per-operation rounding of c10::Half.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libtpo_oracle.so")
_lib = None

_DT = {np.dtype(np.float32): 0, np.dtype(np.float64): 1, np.dtype(np.float16): 2}

P = ctypes.c_void_p
I64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sig = {
            "tpo_ref_chamfer_fwd": [ctypes.c_int, P, P, I64, I64, I64, P, P, P, P],
            "tpo_ref_chamfer_bwd": [ctypes.c_int, P, P, P, P, P, P, I64, I64, I64, P, P, ctypes.c_int],
            "tpo_ref_knn_choose_version": [I64, I64, ctypes.c_int],
            "tpo_ref_knn_fwd": [ctypes.c_int, P, P, P, P, I64, I64, I64, I64, I64, ctypes.c_int,
                                ctypes.c_int, P, P],
            "tpo_ref_knn_bwd": [ctypes.c_int, P, P, P, P, P, ctypes.c_int, P, I64, I64, I64, I64,
                                I64, P, P, ctypes.c_int],
            "tpo_ref_fps_block_size": [I64],
            "tpo_ref_fps": [ctypes.c_int, P, I64, I64, I64, P],
            "tpo_ref_fps_rank": [I64, I64],
            "tpo_ref_gather_fwd": [ctypes.c_int, P, P, I64, I64, I64, I64, P],
            "tpo_ref_gather_bwd": [ctypes.c_int, P, P, I64, I64, I64, I64, P, ctypes.c_int],
            "tpo_ref_emd_fwd": [ctypes.c_int, P, P, I64, I64, I64, P, P],
            "tpo_ref_emd_bwd": [ctypes.c_int, P, P, P, P, I64, I64, I64, P, P],
            "tpo_ref_f32_to_f16_array": [P, P, I64],
            "tpo_ref_f16_to_f32_array": [P, P, I64],
            "tpo_ref_f16_round_check": [],
            "tpo_cpu_knn_fwd": [ctypes.c_int, P, P, P, P, I64, I64, I64, I64, I64, ctypes.c_int,
                                P, P, ctypes.c_int],
            "tpo_cpu_knn_bwd": [ctypes.c_int, P, P, P, P, P, ctypes.c_int, P, I64, I64, I64, I64,
                                I64, P, P, ctypes.c_int],
            "tpo_cpu_fps": [ctypes.c_int, P, I64, I64, I64, P, ctypes.c_int],
            "tpo_cpu_gather_fwd": [ctypes.c_int, P, P, I64, I64, I64, I64, P],
            "tpo_cpu_gather_bwd": [ctypes.c_int, P, P, I64, I64, I64, I64, P],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        L.tpo_ref_fps_rank.restype = I64
        L.tpo_ref_f16_round_check.restype = I64
        _lib = L
    return _lib


def _c(a, dtype=None):
    a = np.asarray(a)
    a = np.ascontiguousarray(a if dtype is None else a.astype(dtype, copy=False))
    return a


def _p(a):
    return a.ctypes.data_as(P)


def _dt(a):
    try:
        return _DT[a.dtype]
    except KeyError as e:
        raise TypeError(f"oracle: unsupported dtype {a.dtype}") from e


def _check(rc, name):
    if rc != 0:
        raise ValueError(f"oracle {name} returned {rc}")


def f32_to_f16_bits(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().tpo_ref_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h):
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().tpo_ref_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def f16_round_check():
    """Float bit patterns where the direct binary16 rounding differs from the
    encode/decode pair (0 expected)."""
    return int(lib().tpo_ref_f16_round_check())


def chamfer_fwd(xyz1, xyz2):
    """chamfer.cu:169-198 -> (dist1, dist2, idx1 int32, idx2 int32)."""
    xyz1, xyz2 = _c(xyz1), _c(xyz2)
    assert xyz1.dtype == xyz2.dtype
    B, N, _ = xyz1.shape
    M = xyz2.shape[1]
    d1 = np.empty((B, N), xyz1.dtype)
    d2 = np.empty((B, M), xyz1.dtype)
    i1 = np.empty((B, N), np.int32)
    i2 = np.empty((B, M), np.int32)
    _check(lib().tpo_ref_chamfer_fwd(_dt(xyz1), _p(xyz1), _p(xyz2), B, N, M, _p(d1), _p(d2),
                                     _p(i1), _p(i2)), "chamfer_fwd")
    return d1, d2, i1, i2


def chamfer_bwd(xyz1, xyz2, idx1, idx2, gd1, gd2, accum_f64=False):
    """chamfer.cu:236-271 -> (grad_xyz1, grad_xyz2)."""
    xyz1, xyz2 = _c(xyz1), _c(xyz2)
    idx1, idx2 = _c(idx1, np.int32), _c(idx2, np.int32)
    gd1, gd2 = _c(gd1, xyz1.dtype), _c(gd2, xyz1.dtype)
    B, N, _ = xyz1.shape
    M = xyz2.shape[1]
    g1 = np.empty_like(xyz1)
    g2 = np.empty_like(xyz2)
    _check(lib().tpo_ref_chamfer_bwd(_dt(xyz1), _p(xyz1), _p(xyz2), _p(idx1), _p(idx2), _p(gd1),
                                     _p(gd2), B, N, M, _p(g1), _p(g2), int(accum_f64)),
           "chamfer_bwd")
    return g1, g2


def knn_choose_version(D, K, version=-1):
    return lib().tpo_ref_knn_choose_version(D, K, version)


def knn_fwd(p1, p2, len1=None, len2=None, norm=2, K=1, version=-1):
    """knn.cu:295-398 (raw, unsorted op output) -> (idxs int64, dists)."""
    p1, p2 = _c(p1), _c(p2)
    N, P1, D = p1.shape
    P2 = p2.shape[1]
    len1 = _c(np.full(N, P1) if len1 is None else len1, np.int64)
    len2 = _c(np.full(N, P2) if len2 is None else len2, np.int64)
    idxs = np.empty((N, P1, K), np.int64)
    dists = np.empty((N, P1, K), p1.dtype)
    _check(lib().tpo_ref_knn_fwd(_dt(p1), _p(p1), _p(p2), _p(len1), _p(len2), N, P1, P2, D, K,
                                 norm, version, _p(idxs), _p(dists)), "knn_fwd")
    return idxs, dists


def knn_bwd(p1, p2, len1, len2, idxs, norm, grad_dists, accum_f64=False):
    """knn.cu:469-534 -> (grad_p1, grad_p2)."""
    p1, p2 = _c(p1), _c(p2)
    N, P1, D = p1.shape
    P2 = p2.shape[1]
    K = idxs.shape[2]
    len1, len2 = _c(len1, np.int64), _c(len2, np.int64)
    idxs = _c(idxs, np.int64)
    grad_dists = _c(grad_dists, p1.dtype)
    g1 = np.empty_like(p1)
    g2 = np.empty_like(p2)
    _check(lib().tpo_ref_knn_bwd(_dt(p1), _p(p1), _p(p2), _p(len1), _p(len2), _p(idxs), norm,
                                 _p(grad_dists), N, P1, P2, D, K, _p(g1), _p(g2),
                                 int(accum_f64)), "knn_bwd")
    return g1, g2


def fps_block_size(n):
    return lib().tpo_ref_fps_block_size(n)


def fps_rank(k, n):
    return lib().tpo_ref_fps_rank(k, n)


def fps(points, nsamples):
    """fps.cu:273-315 -> idx (B, nsamples) int64."""
    points = _c(points)
    B, N, _ = points.shape
    idx = np.empty((B, nsamples), np.int64)
    _check(lib().tpo_ref_fps(_dt(points), _p(points), B, N, nsamples, _p(idx)), "fps")
    return idx


def gather_fwd(points, idx):
    """fps.cu:318-357 -> (B, C, M)."""
    points = _c(points)
    idx = _c(idx, np.int64)
    B, C, N = points.shape
    M = idx.shape[1]
    out = np.empty((B, C, M), points.dtype)
    _check(lib().tpo_ref_gather_fwd(_dt(points), _p(points), _p(idx), B, C, N, M, _p(out)),
           "gather_fwd")
    return out


def gather_bwd(grad_out, idx, n, accum_f64=False):
    """fps.cu:360-404 -> (B, C, n)."""
    grad_out = _c(grad_out)
    idx = _c(idx, np.int64)
    B, C, M = grad_out.shape
    out = np.empty((B, C, n), grad_out.dtype)
    _check(lib().tpo_ref_gather_bwd(_dt(grad_out), _p(grad_out), _p(idx), B, C, n, M, _p(out),
                                    int(accum_f64)), "gather_bwd")
    return out


# --- reference CPU kernels (knn.cpp / fps.cpp semantics) --------------------

def cpu_knn_fwd(p1, p2, len1, len2, K, norm=2, nthreads=1):
    """knn.cpp:30-99 restated -> (idxs int64 sorted ascending, padding -1; dists)."""
    p1, p2 = _c(p1), _c(p2)
    assert p1.dtype == p2.dtype
    N, P1, D = p1.shape
    P2 = p2.shape[1]
    len1, len2 = _c(len1, np.int64), _c(len2, np.int64)
    idxs = np.empty((N, P1, K), np.int64)
    dists = np.empty((N, P1, K), p1.dtype)
    _check(lib().tpo_cpu_knn_fwd(_dt(p1), _p(p1), _p(p2), _p(len1), _p(len2), N, P1, P2, D, K,
                                 norm, _p(idxs), _p(dists), nthreads), "cpu_knn_fwd")
    return idxs, dists


def cpu_knn_bwd(p1, p2, len1, len2, idxs, norm, grad_dists, nthreads=1):
    """knn.cpp:104-164 restated -> (grad_p1, grad_p2)."""
    p1, p2 = _c(p1), _c(p2)
    N, P1, D = p1.shape
    P2 = p2.shape[1]
    K = idxs.shape[2]
    len1, len2 = _c(len1, np.int64), _c(len2, np.int64)
    idxs = _c(idxs, np.int64)
    grad_dists = _c(grad_dists, p1.dtype)
    g1 = np.empty_like(p1)
    g2 = np.empty_like(p2)
    _check(lib().tpo_cpu_knn_bwd(_dt(p1), _p(p1), _p(p2), _p(len1), _p(len2), _p(idxs), norm,
                                 _p(grad_dists), N, P1, P2, D, K, _p(g1), _p(g2), nthreads),
           "cpu_knn_bwd")
    return g1, g2


def cpu_fps(points, nsamples, nthreads=1):
    """fps.cpp:18-88 restated (CPU semantics) -> idx (B, nsamples) int64."""
    points = _c(points)
    B, N, _ = points.shape
    idx = np.empty((B, nsamples), np.int64)
    _check(lib().tpo_cpu_fps(_dt(points), _p(points), B, N, nsamples, _p(idx), nthreads),
           "cpu_fps")
    return idx


def cpu_gather_fwd(points, idx):
    """fps.cpp:91-115 restated -> (B, C, M)."""
    points = _c(points)
    idx = _c(idx, np.int64)
    B, C, N = points.shape
    M = idx.shape[1]
    out = np.empty((B, C, M), points.dtype)
    _check(lib().tpo_cpu_gather_fwd(_dt(points), _p(points), _p(idx), B, C, N, M, _p(out)),
           "cpu_gather")
    return out


def cpu_gather_bwd(grad_out, idx, n):
    """fps.cpp:118-141 restated -> (B, C, n)."""
    grad_out = _c(grad_out)
    idx = _c(idx, np.int64)
    B, C, M = grad_out.shape
    out = np.empty((B, C, n), grad_out.dtype)
    _check(lib().tpo_cpu_gather_bwd(_dt(grad_out), _p(grad_out), _p(idx), B, C, n, M, _p(out)),
           "cpu_gather_bwd")
    return out


def emd_fwd(xyz1, xyz2):
    """emd.cu:18-230 -> (cost[B] before the division by n, match[B, m, n])."""
    xyz1, xyz2 = _c(xyz1), _c(xyz2)
    assert xyz1.dtype == xyz2.dtype
    B, n, _ = xyz1.shape
    m = xyz2.shape[1]
    cost = np.empty((B,), xyz1.dtype)
    match = np.zeros((B, m, n), xyz1.dtype)
    _check(lib().tpo_ref_emd_fwd(_dt(xyz1), _p(xyz1), _p(xyz2), B, n, m, _p(cost), _p(match)),
           "emd_fwd")
    return cost, match


def emd_bwd(grad_cost, xyz1, xyz2, match):
    """emd.cu:234-303 -> (grad_xyz1, grad_xyz2)."""
    xyz1, xyz2 = _c(xyz1), _c(xyz2)
    grad_cost, match = _c(grad_cost, xyz1.dtype), _c(match, xyz1.dtype)
    B, n, _ = xyz1.shape
    m = xyz2.shape[1]
    g1 = np.empty_like(xyz1)
    g2 = np.empty_like(xyz2)
    _check(lib().tpo_ref_emd_bwd(_dt(xyz1), _p(grad_cost), _p(xyz1), _p(xyz2), _p(match), B, n,
                                 m, _p(g1), _p(g2)), "emd_bwd")
    return g1, g2
