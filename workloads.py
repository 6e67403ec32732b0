"""Synthetic inputs for the BASELINE.json configurations.

All inputs are drawn on the CPU from a seeded torch.Generator and can then be
moved to the GPU, so the same seed gives the same bits everywhere.

  c1  chamfer, B=1, N=M=128, uniform [0,1)^3
  c2  chamfer, B=32, N=M=8192, mixture of 8 Gaussians (sigma 0.1, centres
      uniform in [-1,1]^3), p2 = permuted p1 + N(0, 0.01) jitter
  c3  knn_points, B=8, P1=P2=16384, D=3, K=16, points on the unit sphere with
      N(0, 0.02) radial noise, ragged lengths uniform in [8192, 16384]
  c4  FPS B=16, N=65536 -> 4096; 90% uniform [-1,1]^3, 10% in a sigma=0.05
      Gaussian blob; then gather_points of a (16, 64, 65536) N(0,1) feature map
  c5  high-D knn, B=4, 4096 x 65536, D=128, K=32, rows L2-normalised
  emd earth mover's distance, B=16, N=M=2048, N(0,1)^3: the reference
      benchmark's generator (benchmark_flops.py:39-49) at the size of its
      published EMD rows (README.md:275,311-314)
"""
from __future__ import annotations

import torch


def _g(seed: int) -> torch.Generator:
    return torch.Generator("cpu").manual_seed(seed)


def chamfer_c1(seed: int = 1, dtype=torch.float32):
    g = _g(seed)
    p1 = torch.rand(1, 128, 3, generator=g)
    p2 = torch.rand(1, 128, 3, generator=g)
    return p1.to(dtype), p2.to(dtype)


def chamfer_c2(seed: int = 2, B: int = 32, N: int = 8192, dtype=torch.float32):
    g = _g(seed)
    centres = torch.rand(B, 8, 3, generator=g) * 2 - 1
    pick = torch.randint(0, 8, (B, N), generator=g)
    p1 = torch.gather(centres, 1, pick[..., None].expand(-1, -1, 3))
    p1 = p1 + 0.1 * torch.randn(B, N, 3, generator=g)
    perm = torch.stack([torch.randperm(N, generator=g) for _ in range(B)])
    p2 = torch.gather(p1, 1, perm[..., None].expand(-1, -1, 3))
    p2 = p2 + 0.01 * torch.randn(B, N, 3, generator=g)
    return p1.to(dtype), p2.to(dtype)


def _sphere(g, B, P):
    d = torch.randn(B, P, 3, generator=g)
    d = d / d.norm(dim=-1, keepdim=True)
    r = 1 + 0.02 * torch.randn(B, P, 1, generator=g)
    return d * r


def knn_c3(seed: int = 3, B: int = 8, P: int = 16384, lo: int = 8192, dtype=torch.float32):
    g = _g(seed)
    p1 = _sphere(g, B, P)
    p2 = _sphere(g, B, P)
    l1 = torch.randint(lo, P + 1, (B,), generator=g)
    l2 = torch.randint(lo, P + 1, (B,), generator=g)
    return p1.to(dtype), p2.to(dtype), l1, l2


def fps_c4(seed: int = 4, B: int = 16, N: int = 65536, origin_blob: bool = False,
           dtype=torch.float32):
    g = _g(seed)
    n_blob = N // 10
    uni = torch.rand(B, N - n_blob, 3, generator=g) * 2 - 1
    if origin_blob:
        c = torch.zeros(B, 1, 3)
    else:
        c = torch.rand(B, 1, 3, generator=g) * 2 - 1
    blob = c + 0.05 * torch.randn(B, n_blob, 3, generator=g)
    pts = torch.cat([uni, blob], 1)
    perm = torch.stack([torch.randperm(N, generator=g) for _ in range(B)])
    pts = torch.gather(pts, 1, perm[..., None].expand(-1, -1, 3))
    return pts.to(dtype)


def gather_c4(seed: int = 5, B: int = 16, C: int = 64, N: int = 65536, M: int = 4096):
    g = _g(seed)
    feats = torch.randn(B, C, N, generator=g)
    grad_out = torch.randn(B, C, M, generator=g)
    return feats, grad_out


def knn_c5(seed: int = 6, B: int = 4, P1: int = 4096, P2: int = 65536, D: int = 128,
           dtype=torch.bfloat16):
    g = _g(seed)
    p1 = torch.randn(B, P1, D, generator=g)
    p2 = torch.randn(B, P2, D, generator=g)
    p1 = p1 / p1.norm(dim=-1, keepdim=True)
    p2 = p2 / p2.norm(dim=-1, keepdim=True)
    return p1.to(dtype), p2.to(dtype)


def emd_b16(seed: int = 7, B: int = 16, N: int = 2048, M: int = 2048, dtype=torch.float32):
    g = _g(seed)
    p1 = torch.randn(B, N, 3, generator=g)
    p2 = torch.randn(B, M, 3, generator=g)
    return p1.to(dtype), p2.to(dtype)
