"""Product paths chosen by size, run at sizes that select them, against the
oracle -- plus the KNN backward at config 3 and every query row of config 5.

  Chamfer forward, float and half: a cloud above 8192 points (the other at
    least 2048) takes the grid sort that streams its cloud from memory, one
    workgroup per cloud (chamfer_grid_sort_kernel<T, 0>).  B = 8 and 16 run
    the batch-per-XCD block order, B = 1, 2 and 3 the plain order; one case
    stretches a cloud with far outliers, so the sort trims its box.  Every
    row of both directions, distances and first-index argmin, bit for bit
    (chamfer.cu:36-167 serves every size with one kernel).
  KNN forward, float D = 3: reference clouds of 16385-32768 points and
    query clouds above 16384 take the streamed grid binning
    (kg_bin<.., 0>); raw MinK slots bit for bit, sorted rows equal to the
    reference module's sort of the oracle's rows (knn/__init__.py:111-131).
  KNN backward at config 3 in full (knn.cu:400-466), both norms.
  Config 5 (B=4, 4096 x 65536, D=128, K=32): every query row of the
    bfloat16 matrix-core path against a float64 brute force on the GPU, and
    every row of the float32 widening (the reference's V0, knn.cu:16-60)
    against the oracle, one cloud per test.
"""
import numpy as np
import pytest
import torch

import workloads
from tests.test_knn_gpu import _module_sort, assert_same, raw

pytestmark = pytest.mark.gpu


def np_(t):
    return t.detach().cpu().numpy()


def assert_bits(got, ref, what):
    got, ref = np.asarray(got), np.asarray(ref)
    assert got.shape == ref.shape and got.dtype == ref.dtype, what
    same = got.view(np.uint8).reshape(got.shape + (-1,)) == \
        ref.view(np.uint8).reshape(ref.shape + (-1,))
    bad = int((~same.all(-1)).sum())
    assert bad == 0, f"{what}: {bad} of {got.size} differ"


# ------------------------------------------------------------------ Chamfer

def _mixture(g, B, n):
    # config 2's distribution: 8 Gaussian blobs, sigma 0.1
    cen = torch.rand(B, 8, 3, generator=g) * 2 - 1
    pick = torch.randint(0, 8, (B, n), generator=g)
    return torch.gather(cen, 1, pick[..., None].expand(-1, -1, 3)) + \
        0.1 * torch.randn(B, n, 3, generator=g)


def _chamfer_case(kind, B, N, M, g):
    if kind == "mixture":
        return _mixture(g, B, N), _mixture(g, B, M)
    if kind == "uniform":
        return torch.rand(B, N, 3, generator=g), torch.rand(B, M, 3, generator=g)
    if kind == "outlier":  # a tight blob plus far points: the sort trims the box
        p1 = 0.05 * torch.randn(B, N, 3, generator=g)
        p2 = 0.05 * torch.randn(B, M, 3, generator=g)
        p1[:, :6] = torch.tensor([[1e4, 0, 0], [-1e4, 0, 0], [0, 1e4, 0], [0, -1e4, 0],
                                  [0, 0, 1e4], [0, 0, -1e4]])
        p2[:, -3:] = torch.tensor([[3e3, 3e3, 0], [0, -3e3, 3e3], [-3e3, 0, -3e3]])
        return p1, p2
    raise ValueError(kind)


CHAMFER_CASES = [
    ("mixture", 2, 20000, 12000),
    ("mixture", 1, 65536, 65536),
    ("mixture", 8, 16384, 16384),
    ("uniform", 8, 12000, 3000),
    ("uniform", 8, 3000, 12000),
    ("uniform", 16, 9000, 2048),
    ("uniform", 3, 12000, 3000),
    ("outlier", 2, 12000, 9000),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("kind,B,N,M", CHAMFER_CASES)
def test_chamfer_streamed_grid_sort_every_row(tpo, O, dev, kind, B, N, M, dtype):
    assert max(N, M) > 8192 and min(N, M) >= 2048  # the streamed sort's domain
    g = torch.Generator().manual_seed(B * 7919 + N + 3 * M + len(kind))
    p1, p2 = (t.to(dtype) for t in _chamfer_case(kind, B, N, M, g))
    print(f"chamfer streamed sort {kind} B={B} N={N} M={M} {dtype}", flush=True)
    d1, d2, i1, i2 = torch.ops.torch_point_ops_chamfer.chamfer_forward(p1.to(dev), p2.to(dev))
    e1, e2, j1, j2 = O.chamfer_fwd(np_(p1), np_(p2))
    assert_bits(np_(d1), e1, "dist1")
    assert_bits(np_(d2), e2, "dist2")
    assert_bits(np_(i1), j1, "idx1")
    assert_bits(np_(i2), j2, "idx2")
    # the fused loss runs the same forward
    loss, k1, k2 = torch.ops.torch_point_ops_chamfer.chamfer_loss_forward(
        p1.to(dev), p2.to(dev), True)
    assert_bits(np_(k1), j1, "loss idx1")
    assert_bits(np_(k2), j2, "loss idx2")
    want = e1.astype(np.float64).mean() + e2.astype(np.float64).mean()
    if np.isinf(want):  # half distances of the far outliers overflow to inf
        assert float(loss) == want
    else:
        assert abs(float(loss) - want) <= (1e-3 if dtype == torch.float16 else 1e-5) * want


# --------------------------------------------------------------------- KNN

def _sphere(g, B, P):
    d = torch.randn(B, P, 3, generator=g)
    d = d / d.norm(dim=-1, keepdim=True)
    return d * (1 + 0.02 * torch.randn(B, P, 1, generator=g))


def _knn_case(kind, g):
    if kind == "long_refs":  # references 16385-30000: the streamed reference binning
        N, P1, P2 = 3, 3000, 30000
        p1, p2 = _sphere(g, N, P1), _sphere(g, N, P2)
        return p1, p2, torch.tensor([P1, 2999, 1500]), torch.tensor([P2, 16385, 16384])
    if kind == "long_refs_clusters":
        N, P1, P2 = 2, 2500, 32768
        cen = torch.rand(N, 6, 3, generator=g) * 2 - 1
        pick = lambda n: cen[torch.arange(N)[:, None], torch.randint(0, 6, (N, n), generator=g)]
        p1 = pick(P1) + 0.02 * torch.randn(N, P1, 3, generator=g)
        p2 = pick(P2) + 0.02 * torch.randn(N, P2, 3, generator=g)
        return p1, p2, torch.tensor([P1, 2400]), torch.tensor([P2, 20001])
    if kind == "long_queries":  # queries above 16384: the streamed query ordering
        N, P = 2, 20000
        p1, p2 = _sphere(g, N, P), _sphere(g, N, P)
        return p1, p2, torch.tensor([P, 16385]), torch.tensor([P, 17000])
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["long_refs", "long_refs_clusters", "long_queries"])
@pytest.mark.parametrize("K,norm,version", [(16, 2, -1), (1, 2, -1), (32, 2, -1), (5, 1, -1),
                                            (16, 2, 0)])
def test_knn_streamed_grid_binning_every_row(tpo, O, dev, kind, K, norm, version):
    g = torch.Generator().manual_seed(K * 101 + norm + len(kind))
    p1, p2, l1, l2 = _knn_case(kind, g)
    print(f"knn streamed binning {kind} P1={p1.shape[1]} P2={p2.shape[1]} K={K} "
          f"norm={norm} version={version}", flush=True)
    idx, d = raw(p1, p2, l1, l2, norm, K, version, dev)
    ei, ed = O.knn_fwd(np_(p1), np_(p2), np_(l1), np_(l2), norm=norm, K=K, version=version)
    assert_same(np_(idx), ei)
    assert_same(np_(d), ed)
    if K >= 2:
        a, b, la, lb = p1.to(dev), p2.to(dev), l1.to(dev), l2.to(dev)
        si, sd = tpo.knn_points(a, b, la, lb, norm=norm, K=K, version=version)
        wi, wd = _module_sort(torch.from_numpy(ei).to(dev), torch.from_numpy(ed).to(dev), lb, K)
        assert torch.equal(si, wi) and torch.equal(sd, wd)


@pytest.mark.parametrize("norm", [2, 1])
def test_knn_backward_config3_every_row(tpo, O, dev, norm):
    p1, p2, l1, l2 = workloads.knn_c3()
    print(f"knn backward config 3 norm={norm}", flush=True)
    a, b, la, lb = p1.to(dev), p2.to(dev), l1.to(dev), l2.to(dev)
    idx, _ = torch.ops.torch_point_ops_knn.knn_forward(a, b, la, lb, norm, 16, -1)
    gd = torch.rand(p1.shape[0], p1.shape[1], 16, generator=torch.Generator().manual_seed(31))
    g1, g2 = torch.ops.torch_point_ops_knn.knn_backward(a, b, la, lb, idx, norm, gd.to(dev))
    e1, e2 = O.knn_bwd(np_(p1), np_(p2), np_(l1), np_(l2), np_(idx), norm, np_(gd),
                       accum_f64=True)
    for got, ref in ((np_(g1), e1), (np_(g2), e2)):
        err = np.abs(got.astype(np.float64) - ref.astype(np.float64)).max()
        assert err <= 1e-5 * np.abs(ref.astype(np.float64)).max(), err
        assert (got[ref == 0] == 0).all()  # rows no slot touches stay exactly zero


# ------------------------------------------------------------------ config 5

_C5 = {}


def _c5_forward(dev, dtype):
    if dtype not in _C5:
        q, r = workloads.knn_c5()
        if dtype == torch.float32:
            q, r = q.float(), r.float()
        B, P1 = q.shape[:2]
        la = torch.full((B,), P1)
        lb = torch.full((B,), r.shape[1])
        _C5.clear()
        _C5[dtype] = (q, r, la, lb) + tuple(raw(q, r, la, lb, 2, 32, -1, dev))
    return _C5[dtype]


def test_bf16_config5_every_row(tpo, dev):
    """All 4 x 4096 rows against float64 squared distances of the bfloat16
    inputs, computed on the GPU 512 rows at a time.  Membership of the 32
    nearest is exact outside an error band around the 32nd distance that
    bounds the float computation; order ascending; distances agree to the
    bfloat16 rounding (the band rule of test_knn_gpu.check_bf16_knn)."""
    q, r, _, _, idx, d = _c5_forward(dev, torch.bfloat16)
    B, P1, D = q.shape
    K = 32
    qd, rd = q.to(dev, torch.float64), r.to(dev, torch.float64)
    qq, rr = (qd * qd).sum(-1), (rd * rd).sum(-1)
    for n in range(B):
        rmax = float(rr[n].max())
        rt = rd[n].T.contiguous()
        for c0 in range(0, P1, 512):
            rows = slice(c0, c0 + 512)
            ex = (qq[n, rows, None] + rr[n, None]) - 2.0 * (qd[n, rows] @ rt)
            got = idx[n, rows]
            s = got.sort(-1).values
            assert int(s[:, 0].min()) >= 0 and int(s[:, -1].max()) < r.shape[1]
            assert bool((s[:, 1:] != s[:, :-1]).all()), "a reference appears twice"
            kth = ex.topk(K, dim=1, largest=False).values[:, K - 1:K]
            qr = qq[n, rows, None]
            band = 8 * (D + 4) * 2.0 ** -24 * (qr + rmax + 2 * (qr * rmax).sqrt())
            gd = ex.gather(1, got)
            assert bool((gd <= kth + band).all()), f"cloud {n} rows {c0}+: outside the 32 nearest"
            must = ex < (kth - band)
            has = torch.zeros_like(must).scatter_(1, got, True)
            assert bool((~must | has).all()), f"cloud {n} rows {c0}+: a clear neighbour missing"
            dd = d[n, rows].to(torch.float64)
            assert bool((dd[:, 1:] >= dd[:, :-1]).all()), "not sorted ascending"
            assert torch.allclose(dd, gd, rtol=2 ** -7, atol=1e-6 + float(band.max()))


@pytest.mark.parametrize("n", [0, 1, 2, 3])
def test_float_config5_shape_every_row_vs_oracle(tpo, O, dev, n):
    """Config 5 widened to float32 with the reference's V0 semantics: every
    row of cloud n, raw MinK slots bit for bit (each row depends only on its
    query and the reference cloud)."""
    q, r, la, lb, idx, d = _c5_forward(dev, torch.float32)
    print(f"config-5 float cloud {n}", flush=True)
    ei, ed = O.knn_fwd(np_(q[n:n + 1]), np_(r[n:n + 1]), np_(la[n:n + 1]), np_(lb[n:n + 1]),
                       norm=2, K=32)
    assert_same(np_(idx[n:n + 1]), ei)
    assert_same(np_(d[n:n + 1]), ed)
