"""KNN on the GPU vs the oracle: the raw op output (the reference's MinK slot
layout, padding rules and distances) bit for bit, plus knn_points/knn_gather
and the reference test suite's semantics (tests/test_knn.py)."""
import numpy as np
import pytest
import torch

import workloads

pytestmark = pytest.mark.gpu


def np_(t):
    return t.detach().cpu().numpy()


def assert_same(got, ref):
    """Bit for bit (so -0.0 and +0.0 differ); any NaN matches any NaN, since
    the bits of a NaN the oracle makes on the CPU are the CPU's."""
    got, ref = np.asarray(got), np.asarray(ref)
    assert got.shape == ref.shape and got.dtype == ref.dtype
    if got.dtype.kind == "f":
        u = np.dtype(f"u{got.dtype.itemsize}")
        same = (got.view(u) == ref.view(u)) | (np.isnan(got) & np.isnan(ref))
    else:
        same = got == ref
    assert same.all(), f"{np.sum(~same)} of {got.size} differ"


def raw(p1, p2, l1, l2, norm, K, version, dev):
    return torch.ops.torch_point_ops_knn.knn_forward(p1.to(dev), p2.to(dev), l1.to(dev),
                                                     l2.to(dev), norm, K, version)


CASES = [
    # dtype, N, P1, P2, D, K, norm, version
    (torch.float32, 2, 100, 300, 3, 16, 2, -1),
    (torch.float32, 3, 257, 129, 3, 1, 2, -1),
    (torch.float32, 2, 64, 64, 3, 2, 2, -1),   # V3, sorted pair
    (torch.float32, 2, 64, 64, 3, 2, 2, 2),    # V2, MinK
    (torch.float32, 2, 70, 90, 3, 3, 1, 3),
    (torch.float32, 2, 70, 90, 3, 32, 2, 2),
    (torch.float32, 2, 50, 80, 3, 7, 2, 0),    # sentinel padding
    (torch.float32, 2, 50, 80, 3, 5, 1, 1),
    (torch.float32, 2, 40, 300, 3, 40, 2, -1),  # K > 32 -> V1, slots in memory
    (torch.float32, 1, 33, 100, 5, 6, 2, -1),
    (torch.float32, 1, 33, 100, 40, 9, 2, -1),   # V0, runtime D
    (torch.float32, 1, 20, 64, 128, 32, 2, -1),  # config-5 shape class in fp32
    (torch.float32, 2, 40, 100, 64, 10, 2, -1),  # D = 64 held in VGPRs
    (torch.float32, 1, 30, 80, 128, 5, 1, -1),
    (torch.float32, 2, 30, 70, 64, 3, 1, 2),     # invalid forced version -> automatic
    (torch.float64, 2, 60, 130, 3, 10, 2, -1),
    (torch.float64, 2, 60, 130, 3, 4, 1, -1),
    (torch.float16, 2, 60, 130, 3, 8, 2, -1),
    (torch.float16, 2, 60, 130, 3, 2, 1, -1),
]


@pytest.mark.parametrize("dtype,N,P1,P2,D,K,norm,version", CASES)
def test_raw_forward_bit_exact(tpo, O, dev, dtype, N, P1, P2, D, K, norm, version):
    g = torch.Generator().manual_seed(P1 * 7 + P2 * 13 + D + K)
    p1 = torch.randn(N, P1, D, generator=g).to(dtype)
    p2 = torch.randn(N, P2, D, generator=g).to(dtype)
    l1 = torch.randint(P1 // 2, P1 + 1, (N,), generator=g)
    l2 = torch.randint(max(1, K // 2), P2 + 1, (N,), generator=g)
    l2[0] = min(P2, max(1, K - 1))  # a cloud shorter than K
    idx, d = raw(p1, p2, l1, l2, norm, K, version, dev)
    ei, ed = O.knn_fwd(np_(p1), np_(p2), np_(l1), np_(l2), norm=norm, K=K, version=version)
    assert_same(np_(idx), ei)
    assert_same(np_(d), ed)


def test_quantised_ties_bit_exact(tpo, O, dev):
    """Coordinates on a coarse grid: many exactly equal distances exercise the
    first-max eviction and the strict-less rule."""
    g = torch.Generator().manual_seed(21)
    p1 = torch.randint(0, 4, (2, 200, 3), generator=g).float()
    p2 = torch.randint(0, 4, (2, 500, 3), generator=g).float()
    l = torch.tensor([200, 150]), torch.tensor([500, 333])
    for K, v in ((16, -1), (2, -1), (2, 2), (4, 3), (5, 0), (40, -1)):
        idx, d = raw(p1, p2, l[0], l[1], 2, K, v, dev)
        ei, ed = O.knn_fwd(np_(p1), np_(p2), np_(l[0]), np_(l[1]), norm=2, K=K, version=v)
        assert_same(np_(idx), ei)
        assert_same(np_(d), ed)


# ---- high-D float with the references sliced over workgroups (few query
# workgroups, long reference clouds): local MinK candidates + exact replay

def _hd_inputs(case, g, D):
    N, P1, P2 = 2, 300, 20000
    if case == "lattice":  # integer coordinates: many exactly equal distances
        p1 = torch.randint(0, 3, (N, P1, D), generator=g).float()
        p2 = torch.randint(0, 3, (N, P2, D), generator=g).float()
    else:
        p1 = torch.randn(N, P1, D, generator=g)
        p2 = torch.randn(N, P2, D, generator=g)
    if case == "descending":  # every reference closer than all before it: lists overflow
        r = p2.norm(dim=-1)
        p2 = torch.gather(p2, 1, r.argsort(dim=1, descending=True)[..., None].expand(-1, -1, D))
        p1 = p1 * 1e-3
    if case == "nonfinite":
        p2[0, 0, 5] = float("nan")       # fill slot 0: the threshold is NaN, nothing is inserted
        p2[1, 3, 0] = float("nan")       # another fill slot: never the maximum
        p2[1, 4, 7] = float("inf")       # an infinite fill distance: evicted first
        p2[0, 8000:8010, 1] = float("nan")
        p2[1, 5000, 2] = float("inf")
        p2[1, 12345, 9] = -float("inf")
        p1[1, 7, 0] = float("nan")       # a NaN query: every distance NaN
        p1[0, 9, 3] = float("inf")
    if case == "duplicates":
        # exact copies of queries among the references: distance 0 (-0.0 under
        # norm 1), in the fill and repeated across slices, so equal values
        # meet in the merge's order and its first-maximum slot rule
        for n in range(N):
            for q in range(0, 40, 3):
                for j in (q % 7, 100 + 37 * q, 5000 + 91 * q, 15000 + 11 * q):
                    p2[n, j] = p1[n, q]
    l1 = torch.tensor([P1, 211])
    l2 = torch.tensor([P2, 9000]) if case != "short" else torch.tensor([P2, 20])
    return p1, p2, l1, l2


@pytest.mark.parametrize("case", ["random", "lattice", "descending", "short", "nonfinite",
                                  "duplicates"])
@pytest.mark.parametrize("D,K,norm", [(128, 32, 2), (128, 9, 1), (64, 16, 2)])
def test_high_d_sliced_forward_bit_exact(tpo, O, dev, case, D, K, norm):
    g = torch.Generator().manual_seed(D + K + norm + len(case))
    p1, p2, l1, l2 = _hd_inputs(case, g, D)
    print(f"high-D sliced case={case} D={D} K={K} norm={norm}", flush=True)
    idx, d = raw(p1, p2, l1, l2, norm, K, -1, dev)
    ei, ed = O.knn_fwd(np_(p1), np_(p2), np_(l1), np_(l2), norm=norm, K=K)
    assert_same(np_(idx), ei)
    assert_same(np_(d), ed)
    a, b, la, lb = p1.to(dev), p2.to(dev), l1.to(dev), l2.to(dev)
    si, sd = tpo.knn_points(a, b, la, lb, norm=norm, K=K)
    wi, wd = _module_sort(torch.from_numpy(ei).to(dev), torch.from_numpy(ed).to(dev), lb, K)
    assert_same(np_(si), np_(wi))
    assert_same(np_(sd), np_(wd))


def _long_cloud_inputs(case, g):
    # long reference clouds (the staged float D=3 sweep over 5000 references,
    # lengths2 ragged, a cloud with a single query row)
    N, P1, P2 = 4, 300, 5000
    if case == "lattice":  # many exactly equal distances
        p1 = torch.randint(0, 6, (N, P1, 3), generator=g).float()
        p2 = torch.randint(0, 6, (N, P2, 3), generator=g).float()
    else:
        p1 = torch.randn(N, P1, 3, generator=g)
        p2 = torch.randn(N, P2, 3, generator=g)
    if case == "nonfinite":
        p2[0, 3, 1] = float("nan")     # in the fill
        p2[1, 700, 0] = float("inf")
        p2[1, 2600:2610, 2] = float("nan")
        p2[2, 4000, 0] = -float("inf")
        p1[2, 5, 1] = float("nan")
        p1[3, 7, 0] = float("inf")
    if case == "descending":  # every reference closer than all before it: all are inserted
        r = p2.norm(dim=-1)
        p2 = torch.gather(p2, 1, r.argsort(dim=1, descending=True)[..., None].expand(-1, -1, 3))
        p1 = p1 * 1e-3
    l1 = torch.tensor([P1, 250, 299, 1])
    l2 = torch.tensor([P2, 1000, 2560, 4321])
    return p1, p2, l1, l2


@pytest.mark.parametrize("case", ["random", "lattice", "nonfinite", "descending"])
@pytest.mark.parametrize("K,norm,version", [(1, 2, -1), (5, 1, -1), (16, 2, -1), (16, 2, 0),
                                            (17, 1, 2), (32, 2, -1), (2, 2, 2)])
def test_long_clouds_forward_bit_exact(tpo, O, dev, case, K, norm, version):
    g = torch.Generator().manual_seed(K * 31 + norm + len(case))
    p1, p2, l1, l2 = _long_cloud_inputs(case, g)
    idx, d = raw(p1, p2, l1, l2, norm, K, version, dev)
    ei, ed = O.knn_fwd(np_(p1), np_(p2), np_(l1), np_(l2), norm=norm, K=K, version=version)
    assert_same(np_(idx), ei)
    assert_same(np_(d), ed)


def _grid_inputs(case, g):
    # float 3-D against clouds of 6000 references: the brute-force prefix
    # plus grid-candidate path (lengths2 ragged around the prefix length)
    N, P1, P2 = 4, 700, 6000
    if case == "sphere":  # config 3's distribution
        def sph(n):
            v = torch.randn(N, n, 3, generator=g)
            v = v / v.norm(dim=-1, keepdim=True)
            return v * (1 + 0.02 * torch.randn(N, n, 1, generator=g))
        p1, p2 = sph(P1), sph(P2)
    elif case == "clusters":  # tight blobs: small, crowded boxes
        cen = torch.rand(N, 6, 3, generator=g) * 2 - 1
        pick = lambda n: cen[torch.arange(N)[:, None], torch.randint(0, 6, (N, n), generator=g)]
        p1 = pick(P1) + 0.01 * torch.randn(N, P1, 3, generator=g)
        p2 = pick(P2) + 0.01 * torch.randn(N, P2, 3, generator=g)
    elif case == "outlier":  # one far reference stretches the grid
        p1 = torch.rand(N, P1, 3, generator=g)
        p2 = torch.rand(N, P2, 3, generator=g)
        p2[:, 4000] = 1e4
        p2[1, 10] = -1e6
    elif case == "flat":  # one axis without extent, integer ties
        p1 = torch.randint(0, 40, (N, P1, 3), generator=g).float() / 8
        p2 = torch.randint(0, 40, (N, P2, 3), generator=g).float() / 8
        p1[..., 2] = 0.5
        p2[..., 2] = 0.5
    else:  # "nonfinite"
        p1 = torch.rand(N, P1, 3, generator=g)
        p2 = torch.rand(N, P2, 3, generator=g)
        p2[0, 5, 1] = float("nan")  # in the fill
        p2[0, 3000, 0] = float("inf")
        p2[1, 100:110, 2] = float("nan")
        p2[2, 5000, 0] = -float("inf")
        p1[2, 5, 1] = float("nan")
        p1[3, 7, 0] = float("inf")
    l1 = torch.tensor([P1, 650, 1, 333])
    l2 = torch.tensor([P2, 300, 2100, 5999])
    return p1, p2, l1, l2


@pytest.mark.parametrize("case", ["sphere", "clusters", "outlier", "flat", "nonfinite"])
@pytest.mark.parametrize("K,norm,version", [(1, 2, -1), (16, 2, -1), (16, 1, 0), (32, 2, 1),
                                            (7, 2, 3), (2, 2, 2)])
def test_grid_candidates_forward_bit_exact(tpo, O, dev, case, K, norm, version):
    g = torch.Generator().manual_seed(K * 17 + norm + 3 * len(case))
    p1, p2, l1, l2 = _grid_inputs(case, g)
    print(f"grid case={case} K={K} norm={norm} version={version}", flush=True)
    idx, d = raw(p1, p2, l1, l2, norm, K, version, dev)
    ei, ed = O.knn_fwd(np_(p1), np_(p2), np_(l1), np_(l2), norm=norm, K=K, version=version)
    assert_same(np_(idx), ei)
    assert_same(np_(d), ed)
    if K >= 2:  # sorted rows: the in-kernel sort equals the module's sort of the raw rows
        a, b, la, lb = p1.to(dev), p2.to(dev), l1.to(dev), l2.to(dev)
        si, sd = tpo.knn_points(a, b, la, lb, norm=norm, K=K, version=version)
        wi, wd = _module_sort(torch.from_numpy(ei).to(dev), torch.from_numpy(ed).to(dev), lb, K)
        assert torch.equal(si, wi)
        assert torch.equal(sd.isnan(), wd.isnan())
        assert torch.equal(torch.nan_to_num(sd), torch.nan_to_num(wd))


@pytest.mark.parametrize("case", ["random", "lattice", "nonfinite"])
@pytest.mark.parametrize("K", [2, 8, 16, 32])
def test_long_clouds_sorted_rows_match_torch_sort(tpo, dev, case, K):
    g = torch.Generator().manual_seed(K + 7 * len(case))
    p1, p2, l1, l2 = _long_cloud_inputs(case, g)
    a, b, la, lb = p1.to(dev), p2.to(dev), l1.to(dev), l2.to(dev)
    for version in (-1, 0, 2):
        for norm in (1, 2):
            si, sd = tpo.knn_points(a, b, la, lb, norm=norm, K=K, version=version)
            ri, rd = torch.ops.torch_point_ops_knn.knn_forward(a, b, la, lb, norm, K, version)
            ei, ed = _module_sort(ri, rd, lb, K)
            assert torch.equal(si, ei), (version, norm)
            assert torch.equal(sd.isnan(), ed.isnan())
            assert torch.equal(torch.nan_to_num(sd), torch.nan_to_num(ed)), (version, norm)


def _module_sort(idxs, dists, lengths2, K):
    # knn_points' sort after the forward (reference knn/__init__.py:111-131)
    if lengths2.min() < K:
        mask = lengths2[:, None] <= torch.arange(K, device=dists.device)[None]
        mask = mask[:, None].expand(-1, dists.shape[1], -1)
        keyed = dists.clone()
        keyed[mask] = torch.tensor(float("inf"), dtype=dists.dtype, device=dists.device)
        ds, order = keyed.sort(dim=2)
        ds[mask] = torch.tensor(0, dtype=dists.dtype, device=dists.device)
    else:
        ds, order = dists.sort(dim=2)
    return idxs.gather(2, order), ds


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16])
@pytest.mark.parametrize("K", [2, 3, 5, 8, 16, 17, 32])
@pytest.mark.parametrize("case", ["lattice", "ragged", "nonfinite", "highd"])
def test_sorted_rows_in_kernel_match_torch_sort(tpo, dev, dtype, K, case):
    # knn_points(return_sorted=True) sorts inside the kernel by replaying
    # torch's network: rows, ties and padding must equal the forward
    # followed by the reference module's torch sort
    g = torch.Generator().manual_seed(K * 7 + len(case))
    D = 3
    if case == "lattice":  # integer points: many exactly equal distances
        p1 = torch.randint(0, 4, (2, 300, 3), generator=g).float()
        p2 = torch.randint(0, 4, (2, 200, 3), generator=g).float()
        l1, l2 = torch.tensor([300, 250]), torch.tensor([200, 120])
    elif case == "ragged":  # one cloud with fewer points than K
        p1 = torch.randn(3, 200, 3, generator=g)
        p2 = torch.randn(3, 150, 3, generator=g).round(decimals=1)
        l1, l2 = torch.tensor([200, 180, 7]), torch.tensor([150, max(1, K // 2), 40])
    elif case == "nonfinite":
        p1 = torch.randn(2, 100, 3, generator=g)
        p2 = torch.randn(2, 120, 3, generator=g)
        p2[0, 3, 1] = float("inf")
        p2[1, 5:9, 0] = float("nan")
        p1[1, 2, 2] = float("inf")
        l1, l2 = torch.tensor([100, 100]), torch.tensor([120, 120])
    else:
        D = 5
        p1 = torch.randint(0, 3, (2, 150, D), generator=g).float()
        p2 = torch.randint(0, 3, (2, 180, D), generator=g).float()
        l1, l2 = torch.tensor([150, 90]), torch.tensor([180, 100])
    a, b = p1.to(dev, dtype), p2.to(dev, dtype)
    la, lb = l1.to(dev), l2.to(dev)
    for version in (-1, 0, 1, 2, 3):
        for norm in (1, 2):
            si, sd = tpo.knn_points(a, b, la, lb, norm=norm, K=K, version=version)
            ri, rd = torch.ops.torch_point_ops_knn.knn_forward(a, b, la, lb, norm, K, version)
            ei, ed = _module_sort(ri, rd, lb, K)
            assert torch.equal(si, ei), (version, norm)
            assert torch.equal(sd.isnan(), ed.isnan())
            assert torch.equal(torch.nan_to_num(sd), torch.nan_to_num(ed)), (version, norm)


def test_sorted_rows_config3_and_gradient(tpo, dev):
    p1, p2, l1, l2 = (t.to(dev) for t in workloads.knn_c3())
    si, sd = tpo.knn_points(p1, p2, l1, l2, K=16)
    ri, rd = torch.ops.torch_point_ops_knn.knn_forward(p1, p2, l1, l2, 2, 16, -1)
    ei, ed = _module_sort(ri, rd, l2, 16)
    assert torch.equal(si, ei) and torch.equal(sd, ed)
    a = p1[:2, :500].clone().requires_grad_(True)
    b = p2[:2, :700].clone().requires_grad_(True)
    la = torch.tensor([500, 300], device=dev)
    lb = torch.tensor([700, 10], device=dev)
    ga, gb = torch.autograd.grad(tpo.knn_points(a, b, la, lb, K=16)[1].square().sum(), (a, b))
    ri, rd = torch.ops.torch_point_ops_knn.knn_forward(a, b, la, lb, 2, 16, -1)
    ra, rb = torch.autograd.grad(_module_sort(ri, rd, lb, 16)[1].square().sum(), (a, b))
    assert torch.allclose(ga, ra, rtol=1e-5, atol=1e-6) and torch.allclose(gb, rb, rtol=1e-5, atol=1e-6)


def _torch_knn_gather(x, idx, lengths):
    # the reference's knn_gather as torch ops (knn/__init__.py:136-183)
    N, M, U = x.shape
    K = idx.shape[2]
    out = x[:, :, None].expand(-1, -1, K, -1).gather(1, idx[..., None].expand(-1, -1, -1, U))
    if lengths.min() < K:
        pad = lengths[:, None] <= torch.arange(K, device=x.device)[None]
        pad = pad[:, None].expand(-1, idx.shape[1], -1)[..., None].expand(-1, -1, -1, U)
        out[pad] = torch.tensor(0, dtype=x.dtype, device=x.device)
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("U,L", [(1, 40), (3, 40), (7, 40), (3, 70001), (5, 33)])
def test_knn_gather_kernel_matches_torch_ops(tpo, dev, dtype, U, L):
    """Small shapes, and 3 x 70001 x 6 rows: the last wave's span of 64 rows
    ends part-way (rows past the end load and store nothing)."""
    g = torch.Generator().manual_seed(U + L)
    N, M, K = 3, 50, 6
    x = torch.randn(N, M, U, generator=g).to(dev, dtype)
    idx = torch.randint(0, M, (N, L, K), generator=g).to(dev)
    lengths = torch.tensor([M, 4, 1], device=dev)
    got = tpo.knn_gather(x, idx, lengths)
    assert torch.equal(got, _torch_knn_gather(x, idx, lengths))
    full = torch.full((N,), M, device=dev)
    assert torch.equal(tpo.knn_gather(x, idx), _torch_knn_gather(x, idx, full))
    if dtype in (torch.float32, torch.float64) and L <= 40:  # (long L: sums of ~8e3 terms)
        a = x.clone().requires_grad_(True)
        b = x.clone().requires_grad_(True)
        w = torch.randn(N, L, K, U, generator=g).to(dev, dtype)
        (ga,) = torch.autograd.grad((tpo.knn_gather(a, idx, lengths) * w).sum(), (a,))
        (gb,) = torch.autograd.grad((_torch_knn_gather(b, idx, lengths) * w).sum(), (b,))
        assert torch.allclose(ga, gb, rtol=1e-6, atol=1e-6)


def test_knn_points_sorted_and_gather(tpo, O, dev):
    g = torch.Generator().manual_seed(22)
    p1 = torch.randn(3, 40, 3, generator=g)
    p2 = torch.randn(3, 60, 3, generator=g)
    l1 = torch.tensor([40, 20, 33])
    l2 = torch.tensor([60, 3, 45])
    idx, d = tpo.knn_points(p1.to(dev), p2.to(dev), l1.to(dev), l2.to(dev), K=5)
    ei, ed = O.knn_fwd(np_(p1), np_(p2), np_(l1), np_(l2), K=5)
    for n in range(3):
        for i in range(int(l1[n])):
            k = min(5, int(l2[n]))
            order = np.argsort(ed[n, i, :k], kind="stable")
            assert np.array_equal(np_(d[n, i, :k]), ed[n, i, :k][order])
            assert np.array_equal(np_(idx[n, i, :k]), ei[n, i, :k][order])
            assert (np_(d[n, i, k:]) == 0).all()
    nn = tpo.knn_gather(p2.to(dev), idx, l2.to(dev))
    for n in range(3):
        for i in range(40):
            for k in range(5):
                if k < int(l2[n]):
                    assert torch.equal(nn[n, i, k], p2[n, int(idx[n, i, k])].to(dev))
                else:
                    assert (nn[n, i, k] == 0).all()


@pytest.mark.parametrize("norm", [1, 2])
@pytest.mark.parametrize("version", [-1, 0])
def test_backward_vs_oracle(tpo, O, dev, norm, version):
    g = torch.Generator().manual_seed(23 + norm)
    p1 = torch.randn(2, 300, 3, generator=g)
    p2 = torch.randn(2, 200, 3, generator=g)
    l1 = torch.tensor([300, 123])
    l2 = torch.tensor([200, 5])
    idx, _ = raw(p1, p2, l1, l2, norm, 8, version, dev)
    gd = torch.rand(2, 300, 8, generator=g)
    g1, g2 = torch.ops.torch_point_ops_knn.knn_backward(
        p1.to(dev), p2.to(dev), l1.to(dev), l2.to(dev), idx, norm, gd.to(dev))
    e1, e2 = O.knn_bwd(np_(p1), np_(p2), np_(l1), np_(l2), np_(idx), norm, np_(gd),
                       accum_f64=True)
    for got, ref in ((np_(g1), e1), (np_(g2), e2)):
        assert np.abs(got - ref).max() <= 1e-5 * max(np.abs(ref).max(), 1e-30)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16])
@pytest.mark.parametrize("D,K,version", [(3, 16, -1), (1, 1, -1), (3, 5, 0), (5, 7, 1),
                                         (8, 32, -1), (3, 40, -1), (2, 256, 0), (3, 300, 0),
                                         (9, 4, -1), (64, 10, -1), (130, 3, 0)])
@pytest.mark.parametrize("norm", [1, 2])
def test_backward_shapes_vs_oracle(tpo, O, dev, dtype, D, K, version, norm):
    """Both backward kernels (a lane per (row, slot) for D <= 8 and K <= 256,
    a wave per row otherwise) on the oracle's raw rows: -1 padding of
    versions 0/1, clouds shorter than K, rows past lengths1, lattice ties
    (norm 1's sign 0 on equal coordinates)."""
    g = torch.Generator().manual_seed(D * 1000 + K * 10 + norm)
    N, P1, P2 = 3, 130, 320
    p1 = torch.randn(N, P1, D, generator=g)
    p2 = torch.randn(N, P2, D, generator=g)
    p1[1] = torch.randint(-2, 3, (P1, D), generator=g).float()
    p2[1] = torch.randint(-2, 3, (P2, D), generator=g).float()
    p1, p2 = p1.to(dtype), p2.to(dtype)
    l1 = torch.tensor([P1, 77, 0])
    l2 = torch.tensor([P2, max(1, K // 2), 5])
    ei, _ = O.knn_fwd(np_(p1), np_(p2), np_(l1), np_(l2), norm=norm, K=K, version=version)
    gd = torch.rand(N, P1, K, generator=g).to(dtype)
    idx = torch.from_numpy(ei)
    g1, g2 = torch.ops.torch_point_ops_knn.knn_backward(
        p1.to(dev), p2.to(dev), l1.to(dev), l2.to(dev), idx.to(dev), norm, gd.to(dev))
    e1, e2 = O.knn_bwd(np_(p1), np_(p2), np_(l1), np_(l2), ei, norm, np_(gd), accum_f64=True)
    tol = 2e-2 if dtype == torch.float16 else (1e-5 if dtype == torch.float32 else 1e-12)
    for got, ref in ((np_(g1), e1), (np_(g2), e2)):
        ref64 = ref.astype(np.float64)
        assert np.abs(got.astype(np.float64) - ref64).max() <= tol * max(np.abs(ref64).max(), 1e-30)
        if dtype != torch.float16:  # untouched rows and points stay exactly zero
            assert (got[ref64 == 0] == 0).all()


@pytest.mark.parametrize("case", ["one_row", "range", "nonfinite"])
def test_backward_accumulation_edge_cases(tpo, O, dev, case):
    """grad_p2 through the bucketed fixed-point accumulation: 48000 terms on
    one reference row (the scale must keep the row sum in range), terms
    spanning 1e-18 .. 1e+18 in one bucket, and infinite / NaN terms (their
    buckets summed in floating point); finite buckets give the same bits on
    every call."""
    g = torch.Generator().manual_seed(len(case))
    N, P1, P2, D, K = 2, 3000, 700, 3, 16
    p1 = torch.randn(N, P1, D, generator=g)
    p2 = torch.randn(N, P2, D, generator=g)
    idx = torch.randint(0, P2, (N, P1, K), generator=g)
    gd = torch.rand(N, P1, K, generator=g)
    if case == "one_row":
        idx[0] = 7
    elif case == "range":
        gd[0, :, :8] *= 1e-18
        gd[0, :, 8:] *= 1e18
        idx[0] = torch.randint(0, 40, (P1, K), generator=g)
    else:
        p1[1, 5, 0] = float("inf")
        p1[1, 9, 2] = float("nan")
    l1 = torch.tensor([P1, P1 - 100])
    l2 = torch.tensor([P2, P2])
    args = (p1.to(dev), p2.to(dev), l1.to(dev), l2.to(dev), idx.to(dev), 2, gd.to(dev))
    g1, g2 = torch.ops.torch_point_ops_knn.knn_backward(*args)
    h1, h2 = torch.ops.torch_point_ops_knn.knn_backward(*args)
    # finite terms are summed exactly (fixed point): the same bits each call;
    # a bucket with a non-finite term sums in floating point, order unspecified
    same = slice(None) if case != "nonfinite" else slice(0, 1)
    assert torch.equal(g2[same], h2[same])
    e1, e2 = O.knn_bwd(np_(p1), np_(p2), np_(l1), np_(l2), np_(idx), 2, np_(gd), accum_f64=True)
    for got, ref in ((np_(g1), e1), (np_(g2), e2)):
        ref64, got64 = ref.astype(np.float64), got.astype(np.float64)
        fin = np.isfinite(ref64)
        assert np.array_equal(np.isnan(got64), np.isnan(ref64))
        assert np.array_equal(got64[np.isinf(ref64)], ref64[np.isinf(ref64)])
        for n in range(N):  # per cloud: cloud 0 of "range" is 1e36 times cloud 1
            f = fin[n]
            scale = max(np.abs(ref64[n][f]).max(), 1e-30)
            assert np.abs(got64[n][f] - ref64[n][f]).max() <= 1e-5 * scale


# ---- the reference test suite's checks (tests/test_knn.py) ----

def torch_reference_knn(p1, p2, K):
    d = ((p1[:, :, None] - p2[:, None]) ** 2).sum(-1)
    sd, si = d.sort(-1)
    return si[..., :K], sd[..., :K]


def test_reference_forward_and_known_values(tpo, dev):
    g = torch.Generator().manual_seed(0)
    p1 = torch.randn(2, 10, 3, generator=g).to(dev)
    p2 = torch.randn(2, 15, 3, generator=g).to(dev)
    for K in (1, 3, 5):
        idx, d = tpo.knn_points(p1, p2, torch.full((2,), 10, device=dev),
                                torch.full((2,), 15, device=dev), K=K)
        ri, rd = torch_reference_knn(p1, p2, K)
        assert torch.allclose(d, rd, atol=1e-5) and torch.equal(idx, ri)
    a = torch.tensor([[[0.0, 0, 0], [1.0, 0, 0]]], device=dev)
    b = torch.tensor([[[0.0, 0, 0], [0.5, 0, 0], [2.0, 0, 0]]], device=dev)
    idx, d = tpo.knn_points(a, b, K=2)
    assert idx.tolist() == [[[0, 1], [1, 0]]]
    assert torch.allclose(d, torch.tensor([[[0.0, 0.25], [0.25, 1.0]]], device=dev))
    q = torch.zeros(1, 1, 3, device=dev)
    r = torch.tensor([[[1.0, 1, 1], [2.0, 0, 0]]], device=dev)
    assert tpo.knn_points(q, r, norm=1, K=2)[1].tolist() == [[[2.0, 3.0]]]
    assert tpo.knn_points(q, r, norm=2, K=2)[1].tolist() == [[[3.0, 4.0]]]


def test_empty_clouds(tpo, dev):
    p1 = torch.randn(2, 10, 3, device=dev)
    e = torch.empty(2, 0, 3, device=dev)
    idx, d = torch.ops.torch_point_ops_knn.knn_forward(
        p1, e, torch.tensor([10, 10], device=dev), torch.tensor([0, 0], device=dev), 2, 3, -1)
    assert idx.shape == (2, 10, 3) and (idx == 0).all() and (d == 0).all()
    idx, d = torch.ops.torch_point_ops_knn.knn_forward(
        e, p1, torch.tensor([0, 0], device=dev), torch.tensor([10, 10], device=dev), 2, 3, -1)
    assert idx.shape == (2, 0, 3)


def test_gradients_and_gradcheck(tpo, dev):
    g = torch.Generator().manual_seed(9)
    for B, N, M, K in ((1, 3, 4, 1), (2, 5, 7, 2), (1, 8, 6, 3), (1, 8, 12, 3)):
        p1 = torch.randn(B, N, 3, generator=g).to(dev).requires_grad_(True)
        p2 = torch.randn(B, M, 3, generator=g).to(dev).requires_grad_(True)
        loss = tpo.knn_points(p1, p2, K=K)[1].mean()
        ga, gb = torch.autograd.grad(loss, (p1, p2))
        ref = torch_reference_knn(p1, p2, K)[1].mean()
        ra, rb = torch.autograd.grad(ref, (p1, p2))
        assert torch.allclose(loss, ref, atol=1e-6)
        assert torch.allclose(ga, ra, atol=1e-4) and torch.allclose(gb, rb, atol=1e-4)
    p1 = torch.randn(1, 4, 3, generator=g, dtype=torch.float64).to(dev).requires_grad_(True)
    p2 = torch.randn(1, 5, 3, generator=g, dtype=torch.float64).to(dev).requires_grad_(True)
    fn = lambda a, b: tpo.knn_points(a, b, K=2, return_sorted=False)[1].sum()  # noqa: E731
    assert torch.autograd.gradcheck(fn, (p1, p2), eps=1e-6, atol=1e-5, rtol=1e-4,
                                    nondet_tol=1e-5, fast_mode=True, check_batched_grad=False)


def test_module_opcheck_compile_precision(tpo, dev):
    from torch.library import opcheck

    g = torch.Generator().manual_seed(10)
    p1 = torch.randn(2, 8, 3, generator=g).to(dev)
    p2 = torch.randn(2, 10, 3, generator=g).to(dev)
    idx, d = tpo.KNearestNeighbors(K=3)(p1, p2)
    assert idx.shape == (2, 8, 3) and d.shape == (2, 8, 3)
    idx, d, nn = tpo.KNearestNeighbors(K=3, return_nn=True)(p1, p2)
    assert nn.shape == (2, 8, 3, 3)
    l = torch.tensor([3], device=dev)
    opcheck(torch.ops.torch_point_ops_knn.knn_forward.default,
            (p1[:1, :3].contiguous(), p2[:1, :3].contiguous(), l, l, 2, 2, -1),
            raise_exception=True)
    opcheck(torch.ops.torch_point_ops_knn.knn_forward_sorted.default,
            (p1[:1, :3].contiguous(), p2[:1, :3].contiguous(), l, l, 2, 2, -1),
            raise_exception=True)
    opcheck(torch.ops.torch_point_ops_knn.knn_gather.default,
            (p2.clone().requires_grad_(True), torch.randint(0, 10, (2, 8, 3), device=dev),
             torch.tensor([10, 2], device=dev)),
            raise_exception=True)
    m = tpo.KNearestNeighbors(K=3).to(dev)
    e, c = m(p1[:1], p2[:1]), torch.compile(m)(p1[:1], p2[:1])
    assert torch.allclose(e[0], c[0]) and torch.allclose(e[1], c[1])
    for dtype in (torch.float16, torch.float32, torch.float64):
        a = p1.detach().to(dtype).clone().requires_grad_(True)
        b = p2.detach().to(dtype).clone().requires_grad_(True)
        idx, d = tpo.knn_points(a, b, K=3)
        assert d.dtype == dtype and idx.dtype == torch.int64
        d.mean().backward()
        assert torch.isfinite(a.grad).all() and torch.isfinite(b.grad).all()
    for v in (0, 1, 2, 3):
        d_auto = tpo.knn_points(p1, p2, K=3)[1]
        d_v = tpo.knn_points(p1, p2, K=3, version=v)[1]
        assert torch.allclose(d_auto, d_v, atol=1e-5)


# ------------------------------------------------------- bfloat16 (extension)
# The reference raises for bfloat16.  The matrix-core kernel (norm 2, D % 8 ==
# 0, D <= 128, K <= 32) computes |q|^2 + |r|^2 - 2 q.r in float; it is checked
# against a float64 brute force on the bfloat16-rounded inputs: membership of
# the K nearest is exact outside an error band around the K-th distance that
# bounds the float computation, order is ascending, distances agree to the
# bfloat16 rounding.  (Parity with the reference is unpinned: it has no
# bfloat16 result to compare with.)

def bf16_expected(q, r, l1, l2, K):
    """float64 squared distances of the bf16 values, per batch (N, P1, P2)."""
    qd = q.to(torch.float64)
    rd = r.to(torch.float64)
    return torch.cdist(qd, rd) ** 2


def check_bf16_knn(idx, d, q, r, l1, l2, K):
    idx, d = idx.cpu(), d.cpu().to(torch.float64)
    exact = bf16_expected(q, r, l1, l2, K)
    D = q.shape[2]
    qq = (q.to(torch.float64) ** 2).sum(-1)
    rr = (r.to(torch.float64) ** 2).sum(-1)
    for n in range(q.shape[0]):
        L1, L2 = int(l1[n]), int(l2[n])
        assert (idx[n, L1:] == 0).all() and (d[n, L1:] == 0).all()
        k_real = min(K, L2)
        assert (idx[n, :L1, k_real:] == 0).all() and (d[n, :L1, k_real:] == 0).all()
        if L1 == 0 or k_real == 0:
            continue
        ex = exact[n, :L1, :L2]
        got = idx[n, :L1, :k_real]
        assert int(got.min()) >= 0 and int(got.max()) < L2
        assert all(len(set(row.tolist())) == k_real for row in got)
        kth = ex.sort(-1).values[:, k_real - 1:k_real]
        # error of the float expansion: a few roundings of |q|^2 + |r|^2 + 2|q.r|
        band = 8 * (D + 4) * 2.0 ** -24 * (qq[n, :L1, None] + rr[n, None, :L2].max() + 2 * (qq[n, :L1, None] * rr[n, None, :L2].max()).sqrt())
        gd = torch.gather(ex, 1, got)
        assert bool((gd <= kth + band).all()), "a returned point is outside the K nearest"
        must = ex < (kth - band)
        has = torch.zeros_like(must)
        has.scatter_(1, got, True)
        assert bool((~must | has).all()), "a point clearly inside the K nearest is missing"
        dd = d[n, :L1, :k_real]
        assert bool((dd[:, 1:] >= dd[:, :-1]).all()), "not sorted ascending"
        assert torch.allclose(dd, gd, rtol=2 ** -7, atol=1e-6 + float(band.max()))


@pytest.mark.parametrize("N,P1,P2,D,K", [(2, 100, 1000, 128, 32), (1, 64, 513, 64, 16),
                                         (2, 50, 300, 40, 5), (1, 33, 90, 8, 1),
                                         (2, 70, 200, 96, 20)])
def test_bf16_matrix_core_knn(tpo, dev, N, P1, P2, D, K):
    g = torch.Generator().manual_seed(N * 1000 + P1 + P2 + D + K)
    q = torch.randn(N, P1, D, generator=g).to(torch.bfloat16)
    r = torch.randn(N, P2, D, generator=g).to(torch.bfloat16)
    l1 = torch.randint(P1 // 2, P1 + 1, (N,), generator=g)
    l2 = torch.randint(K, P2 + 1, (N,), generator=g)
    if N > 1:
        l2[1] = max(1, K // 2)  # fewer references than K
    idx, d = raw(q, r, l1, l2, 2, K, -1, dev)
    assert idx.dtype == torch.int64 and d.dtype == torch.bfloat16
    check_bf16_knn(idx, d, q, r, l1, l2, K)


def test_bf16_equal_distances_take_lower_indices(tpo, dev):
    # every reference point four times: rows 2i, 2i + 1 (neighbours in one
    # tile) and 2P + 2i, 2P + 2i + 1 (another slice); the copies give equal
    # float distances, so each query's list is its nearest point's four copies
    # in index order, then the two lowest copies of its second nearest --
    # exactly, on the rows whose three nearest distinct points are clearly
    # apart (float64 gaps above the error band)
    g = torch.Generator().manual_seed(91)
    B, P1, P, D, K = 2, 256, 3072, 64, 6  # 12288 references: the sampled bound applies
    q = torch.randn(B, P1, D, generator=g).to(torch.bfloat16)
    r0 = torch.randn(B, P, D, generator=g).to(torch.bfloat16)
    r = torch.cat([r0.repeat_interleave(2, 1), r0.repeat_interleave(2, 1)], 1)
    l1 = torch.full((B,), P1, dtype=torch.int64)
    l2 = torch.full((B,), 4 * P, dtype=torch.int64)
    idx, d = raw(q, r, l1, l2, 2, K, -1, dev)
    idx = idx.cpu()
    ex = bf16_expected(q, r0, l1, l2, K)  # (B, P1, P)
    top = ex.sort(-1)
    qq = (q.to(torch.float64) ** 2).sum(-1)
    rmax = (r0.to(torch.float64) ** 2).sum(-1).max(-1).values
    checked = 0
    for n in range(B):
        for row in range(P1):
            v, j = top.values[n, row], top.indices[n, row]
            band = 8 * (D + 4) * 2.0 ** -24 * float((qq[n, row].sqrt() + rmax[n].sqrt()) ** 2)
            if not (v[1] - v[0] > band and v[2] - v[1] > band):
                continue
            a, b = int(j[0]), int(j[1])
            want = [2 * a, 2 * a + 1, 2 * P + 2 * a, 2 * P + 2 * a + 1, 2 * b, 2 * b + 1]
            assert idx[n, row].tolist() == want, (n, row)
            checked += 1
    assert checked > B * P1 // 2
    assert bool((d[..., :4] == d[..., :1]).all())


def test_bf16_rows_the_sampled_bound_leaves_short_are_rerun(tpo, dev):
    # Clouds of >= max(4096, 1536 K) references first bound each query by the
    # 8th smallest of its minimum distances over 64 sampled tiles of 32
    # references (tiles i * (tiles // 64)); only distances under the bound are
    # candidates, and a row left with fewer than K is rerun without it.  Here
    # the first 32 queries of cloud 0 have 8 near copies in 8 different
    # sampled tiles and their next 24 neighbours outside them: their bound
    # admits 8 candidates, so they take the rerun; the other queries have
    # their near points outside the sample and keep the bound.  Cloud 1 has
    # 40000 references, below 1536 K: all its 50 rows take the exact pass.
    # The lists must be the K nearest either way (float64 check).
    g = torch.Generator().manual_seed(17)
    B, P1, P2, D, K = 2, 64, 65536, 64, 32
    l2 = torch.tensor([P2, 40000])
    q = torch.randn(B, P1, D, generator=g)
    q = q / q.norm(dim=-1, keepdim=True)
    r = torch.randn(B, P2, D, generator=g)
    r = r / r.norm(dim=-1, keepdim=True)
    for b in range(B):
        tiles = (int(l2[b]) + 31) // 32
        stride = tiles // 64
        sampled = torch.cat([torch.arange(32) + 32 * stride * i for i in range(64)])
        others = torch.tensor(sorted(set(range(int(l2[b]))) - set(sampled.tolist())))
        pick = others[torch.randperm(len(others), generator=g)]
        for k in range(P1):
            if k < 32:
                slot = 8 * k + torch.arange(8)  # tiles slot % 64, row slot // 64 of the tile
                near = 32 * stride * (slot % 64) + slot // 64
                r[b, near] = q[b, k] + 0.02 * torch.randn(8, D, generator=g)
                mid = pick[24 * k:24 * k + 24]
                r[b, mid] = q[b, k] + 0.06 * torch.randn(24, D, generator=g)
            else:
                spread = pick[24 * k:24 * k + 40]
                r[b, spread] = q[b, k] + 0.04 * torch.randn(40, D, generator=g)
    q, r = q.to(torch.bfloat16), r.to(torch.bfloat16)
    l1 = torch.tensor([P1, 50])
    idx, d = raw(q, r, l1, l2, 2, K, -1, dev)
    check_bf16_knn(idx, d, q, r, l1, l2, K)
    # the same call through the C ABI with a caller workspace, whose rerun
    # counts (after the norms, the 8 slices' lists and the bound's parts)
    # show that exactly the 32 planted rows of cloud 0 and all 50 rows of
    # cloud 1 were rerun
    import ctypes
    from torch_point_ops import _native

    lib = ctypes.CDLL(_native.HIP_LIB)
    P, I = ctypes.c_void_p, ctypes.c_int64
    lib.tpo_knn_fwd.argtypes = [ctypes.c_int, P, P, P, P, I, I, I, I, I, ctypes.c_int,
                                ctypes.c_int, P, P, P, P, I, P]
    lib.tpo_knn_workspace_size.argtypes = [ctypes.c_int, I, I, I, I, I, ctypes.c_int]
    lib.tpo_knn_workspace_size.restype = I
    size = lib.tpo_knn_workspace_size(3, B, P1, P2, D, K, 2)
    ws = torch.zeros(size, dtype=torch.uint8, device=dev)
    qd, rd, l1d, l2d = q.to(dev), r.to(dev), l1.to(dev), l2.to(dev)
    idx2 = torch.empty(B, P1, K, dtype=torch.int64, device=dev)
    d2 = torch.empty(B, P1, K, dtype=torch.bfloat16, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.tpo_knn_fwd(3, qd.data_ptr(), rd.data_ptr(), l1d.data_ptr(), l2d.data_ptr(), B, P1,
                           P2, D, K, 2, -1, idx2.data_ptr(), d2.data_ptr(), None, ws.data_ptr(),
                           size, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(idx2, idx.to(dev)) and torch.equal(d2, d.to(dev))
    up = lambda x: (x + 255) // 256 * 256
    at = up(B * (P1 + 32 * ((P2 + 31) // 32)) * 4) + up(B * P1 * 8 * K * 8) + up(B * P1 * 64 * 4)
    # then the rerun lists and the candidate pass's 16 slices of 128 keys and
    # two counts per query
    assert at + up(B * 4) + up(B * P1 * 4) + up(B * P1 * 16 * 128 * 8) + up(B * P1 * 16 * 2 * 4) == size
    counts = ws[at:at + 4 * B].cpu().view(torch.int32)
    assert counts.tolist() == [32, 50]


@pytest.mark.parametrize("D", [8, 16, 40, 72, 120])
def test_bf16_candidate_pass_dims(tpo, dev, D):
    # the sampled bound and the candidate pass (4096 references, K = 2 so the
    # bound applies) for every operand layout: D % 16 == 8 puts the norm step
    # in the upper half of the last dimension step, else in a step of its own
    g = torch.Generator().manual_seed(300 + D)
    B, P1, P2, K = 2, 96, 4096, 2
    q = torch.randn(B, P1, D, generator=g).to(torch.bfloat16)
    r = torch.randn(B, P2, D, generator=g).to(torch.bfloat16)
    l1 = torch.tensor([P1, 70])
    l2 = torch.tensor([P2, P2])
    idx, d = raw(q, r, l1, l2, 2, K, -1, dev)
    check_bf16_knn(idx, d, q, r, l1, l2, K)


def test_bf16_candidate_regions_wide_overflowed_and_tied(tpo, dev):
    # Clouds of >= 4096 references run the candidate pass: each (query,
    # slice) region holds up to 128 candidates, one register a slice in the
    # merge while every region holds <= 64, two otherwise; an overflowed
    # region, or more than 512 candidates left by the merge's histogram (a
    # mass of equal distances), sends the row to the exact pass.  Here 16
    # slices of 512 references (16 tiles; tiles 4i are sampled; K = 4 so that
    # 8192 references take the bound).  Query 0 of cloud 0 has 100 near
    # points in slice 0 (two registers, no overflow), query 0 of cloud 1 has
    # 200 there (overflow), and query 0 of cloud 2 has 38 exact copies of one
    # near point at the head of every slice (608 equal distances: rerun, and
    # the list must be their K lowest indices).
    import ctypes
    from torch_point_ops import _native
    g = torch.Generator().manual_seed(29)
    B, P1, P2, D, K = 3, 64, 8192, 64, 4
    q = torch.randn(B, P1, D, generator=g)
    q = q / q.norm(dim=-1, keepdim=True)
    r = torch.randn(B, P2, D, generator=g)
    r = r / r.norm(dim=-1, keepdim=True)
    r[0, :100] = q[0, 0] + 0.05 * torch.randn(100, D, generator=g)
    r[1, :200] = q[1, 0] + 0.05 * torch.randn(200, D, generator=g)
    near = q[2, 0] + 0.05 * torch.randn(D, generator=g)
    for sl in range(16):
        r[2, 512 * sl:512 * sl + 38] = near
    q, r = q.to(torch.bfloat16), r.to(torch.bfloat16)
    l1 = torch.full((B,), P1, dtype=torch.int64)
    l2 = torch.full((B,), P2, dtype=torch.int64)
    idx, d = raw(q, r, l1, l2, 2, K, -1, dev)
    check_bf16_knn(idx, d, q, r, l1, l2, K)
    assert idx[2, 0].tolist() == list(range(K))
    assert bool((d[2, 0] == d[2, 0, 0]).all())
    # through the C ABI with a caller workspace: the rerun lists (after the
    # norms, the exact pass's 8 slices of lists, the bound's parts and the
    # rerun counts) hold query 0 of clouds 1 and 2, not of cloud 0 (other
    # rows may fall short of K candidates and join them)
    lib = ctypes.CDLL(_native.HIP_LIB)
    P, I = ctypes.c_void_p, ctypes.c_int64
    lib.tpo_knn_fwd.argtypes = [ctypes.c_int, P, P, P, P, I, I, I, I, I, ctypes.c_int,
                                ctypes.c_int, P, P, P, P, I, P]
    lib.tpo_knn_workspace_size.argtypes = [ctypes.c_int, I, I, I, I, I, ctypes.c_int]
    lib.tpo_knn_workspace_size.restype = I
    size = lib.tpo_knn_workspace_size(3, B, P1, P2, D, K, 2)
    ws = torch.zeros(size, dtype=torch.uint8, device=dev)
    qd, rd, l1d, l2d = q.to(dev), r.to(dev), l1.to(dev), l2.to(dev)
    idx2 = torch.empty(B, P1, K, dtype=torch.int64, device=dev)
    d2 = torch.empty(B, P1, K, dtype=torch.bfloat16, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.tpo_knn_fwd(3, qd.data_ptr(), rd.data_ptr(), l1d.data_ptr(), l2d.data_ptr(), B, P1,
                           P2, D, K, 2, -1, idx2.data_ptr(), d2.data_ptr(), None, ws.data_ptr(),
                           size, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(idx2, idx.to(dev)) and torch.equal(d2, d.to(dev))
    up = lambda x: (x + 255) // 256 * 256
    at = up(B * (P1 + P2) * 4) + up(B * P1 * 8 * K * 8) + up(B * P1 * 64 * 4)
    counts = ws[at:at + 4 * B].cpu().view(torch.int32).tolist()
    rl = ws[at + up(B * 4):at + up(B * 4) + 4 * B * P1].cpu().view(torch.int32).view(B, P1)
    listed = [set(rl[n, :counts[n]].tolist()) for n in range(B)]
    assert 0 not in listed[0] and 0 in listed[1] and 0 in listed[2], (counts, listed)


def test_bf16_knn_points_and_fallbacks(tpo, dev):
    g = torch.Generator().manual_seed(77)
    q = torch.randn(2, 40, 64, generator=g).to(torch.bfloat16).to(dev)
    r = torch.randn(2, 300, 64, generator=g).to(torch.bfloat16).to(dev)
    idx, dists, nn = tpo.KNearestNeighbors(K=8, return_nn=True)(q, r)
    assert dists.dtype == torch.bfloat16 and nn.shape == (2, 40, 8, 64)
    assert bool((dists[..., 1:] >= dists[..., :-1]).all())
    _, ref = tpo.knn_points(q.float(), r.float(), K=8)
    assert torch.allclose(dists.float(), ref, rtol=2 ** -6, atol=1e-3)
    # routes computed in float on the widened values: L1, D not a multiple of 8
    for (D, norm) in ((64, 1), (3, 2)):
        qa = torch.randn(2, 30, D, generator=g).to(torch.bfloat16)
        ra = torch.randn(2, 90, D, generator=g).to(torch.bfloat16)
        l1 = torch.tensor([30, 20])
        l2 = torch.tensor([90, 5])
        i_b, d_b = raw(qa, ra, l1, l2, norm, 6, -1, dev)
        i_f, d_f = raw(qa.float(), ra.float(), l1, l2, norm, 6, -1, dev)
        assert torch.equal(i_b, i_f) and torch.equal(d_b, d_f.to(torch.bfloat16))
    # backward in float, rounded once
    a = q.detach().clone().requires_grad_(True)
    b = r.detach().clone().requires_grad_(True)
    tpo.knn_points(a, b, K=4)[1].float().sum().backward()
    assert a.grad.dtype == torch.bfloat16 and torch.isfinite(a.grad.float()).all()
    assert torch.isfinite(b.grad.float()).all()
