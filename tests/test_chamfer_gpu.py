"""Chamfer on the GPU vs the oracle (bit-exact distances and first-index argmin)
and the reference test suite's semantics (tests/test_chamfer.py)."""
import numpy as np
import pytest
import torch

import workloads

pytestmark = pytest.mark.gpu


def np_(t):
    return t.detach().cpu().numpy()


def assert_bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype
    assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), \
        f"{np.sum(a != b)} of {a.size} differ"


def run_fwd(p1, p2, dev):
    return torch.ops.torch_point_ops_chamfer.chamfer_forward(p1.to(dev), p2.to(dev))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16])
def test_config1_forward_backward_vs_oracle(tpo, O, dev, dtype):
    p1, p2 = workloads.chamfer_c1(dtype=dtype)
    d1, d2, i1, i2 = run_fwd(p1, p2, dev)
    e1, e2, j1, j2 = O.chamfer_fwd(np_(p1), np_(p2))
    assert_bits(np_(d1), e1)
    assert_bits(np_(d2), e2)
    assert np.array_equal(np_(i1), j1) and np.array_equal(np_(i2), j2)
    # backward of ChamferDistance('mean') (grad_dist = 1/N each)
    a = p1.to(dev).requires_grad_(True)
    b = p2.to(dev).requires_grad_(True)
    tpo.ChamferDistance("mean")(a, b).backward()
    g1 = np.full(e1.shape, 1.0 / e1.size, dtype=e1.dtype)
    g2 = np.full(e2.shape, 1.0 / e2.size, dtype=e2.dtype)
    ea, eb = O.chamfer_bwd(np_(p1), np_(p2), j1, j2, g1, g2, accum_f64=True)
    tol = 1e-2 if dtype == torch.float16 else 1e-5
    for got, ref in ((np_(a.grad), ea), (np_(b.grad), eb)):
        scale = max(np.abs(ref).max(), 1e-30)
        assert np.abs(got.astype(np.float64) - ref).max() <= tol * scale


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16])
@pytest.mark.parametrize("B,N,M", [(1, 1, 1), (2, 5, 7), (3, 64, 1), (1, 513, 1000),
                                   (2, 1000, 333), (4, 4097, 2049), (1, 20000, 17)])
def test_forward_bit_exact_random_sizes(tpo, O, dev, dtype, B, N, M):
    g = torch.Generator().manual_seed(B * 1000003 + N * 31 + M)
    p1 = torch.randn(B, N, 3, generator=g).to(dtype)
    p2 = torch.randn(B, M, 3, generator=g).to(dtype)
    d1, d2, i1, i2 = run_fwd(p1, p2, dev)
    e1, e2, j1, j2 = O.chamfer_fwd(np_(p1), np_(p2))
    assert_bits(np_(d1), e1)
    assert_bits(np_(d2), e2)
    assert np.array_equal(np_(i1), j1) and np.array_equal(np_(i2), j2)


def test_duplicates_first_index(tpo, O, dev):
    g = torch.Generator().manual_seed(11)
    p1 = torch.rand(2, 300, 3, generator=g)
    p2 = torch.rand(2, 900, 3, generator=g)
    p2[:, 700] = p2[:, 5]
    p2[:, 333] = p2[:, 5]
    p2[:, 100:200] = p2[:, 0:100]  # whole duplicated range
    d1, _, i1, _ = run_fwd(p1, p2, dev)
    e1, _, j1, _ = O.chamfer_fwd(np_(p1), np_(p2))
    assert np.array_equal(np_(i1), j1)
    assert not np.isin(np_(i1), [333, 700]).any() and not (np_(i1)[:, :] // 100 == 1).any()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.float64])
@pytest.mark.parametrize("B,N,M", [(2, 20000, 17), (1, 70000, 900), (3, 4097, 5000)])
def test_backward_slices_and_two_pass_vs_oracle(tpo, O, dev, dtype, B, N, M):
    # sliced LDS accumulation (several slices per cloud, ragged last slice)
    # and, for 70000 points, the two-pass global-atomic path
    g = torch.Generator().manual_seed(N + M)
    p1 = torch.randn(B, N, 3, generator=g).to(dtype)
    p2 = torch.randn(B, M, 3, generator=g).to(dtype)
    gd1 = torch.rand(B, N, generator=g).to(dtype)
    gd2 = torch.rand(B, M, generator=g).to(dtype)
    _, _, j1, j2 = O.chamfer_fwd(np_(p1), np_(p2))
    ea, eb = O.chamfer_bwd(np_(p1), np_(p2), j1, j2, np_(gd1), np_(gd2), accum_f64=True)
    ga, gb = torch.ops.torch_point_ops_chamfer.chamfer_backward(
        p1.to(dev), p2.to(dev), torch.from_numpy(j1).to(dev), torch.from_numpy(j2).to(dev),
        gd1.to(dev), gd2.to(dev))
    tol = 2e-2 if dtype == torch.float16 else (1e-5 if dtype == torch.float32 else 1e-12)
    for got, ref in ((np_(ga), ea), (np_(gb), eb)):
        assert np.abs(got.astype(np.float64) - ref).max() <= tol * max(np.abs(ref).max(), 1e-30)


# ---- edge cases of the float filter (expanded-form ranking + exact re-scan)
# and of the NaN rule of the reference's 512-reference stages

def assert_same(a, b):
    """Bitwise equality, except that NaN matches NaN whatever its payload."""
    a, b = np.asarray(a), np.asarray(b)
    na, nb = np.isnan(a), np.isnan(b)
    assert np.array_equal(na, nb), f"NaN pattern differs: {np.sum(na != nb)}"
    assert_bits(np.where(na, 0, a).astype(a.dtype), np.where(nb, 0, b).astype(b.dtype))


def check_vs_oracle(O, dev, p1, p2):
    d1, d2, i1, i2 = run_fwd(p1, p2, dev)
    e1, e2, j1, j2 = O.chamfer_fwd(np_(p1), np_(p2))
    assert_same(np_(d1), e1)
    assert_same(np_(d2), e2)
    assert np.array_equal(np_(i1), j1) and np.array_equal(np_(i2), j2)
    return np_(i1), np_(i2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16])
def test_lattice_ties_across_tiles(tpo, O, dev, dtype):
    # shuffled integer lattice; half-integer queries are equidistant from up to
    # 8 lattice points that sit in different tiles and chunks
    g = torch.Generator().manual_seed(21)
    ax = torch.arange(12.0)
    lat = torch.stack(torch.meshgrid(ax, ax, ax, indexing="ij"), -1).reshape(1, -1, 3)
    p2 = lat[:, torch.randperm(lat.shape[1], generator=g)]
    p1 = torch.randint(0, 23, (1, 3000, 3), generator=g).float() / 2
    check_vs_oracle(O, dev, p1.to(dtype), p2.to(dtype))


@pytest.mark.parametrize("offset", [1e2, 1e3, 3e4])
def test_far_from_origin_float(tpo, O, dev, offset):
    # |q|^2 large against the spacing: the filter window admits many tiles and
    # most queries take the exact wave scan; at 3e4 many distances tie exactly
    g = torch.Generator().manual_seed(int(offset))
    p1 = torch.rand(2, 3000, 3, generator=g) + offset
    p2 = torch.rand(2, 2500, 3, generator=g) + offset
    check_vs_oracle(O, dev, p1, p2)


@pytest.mark.parametrize("scale", [1e-10, 1e-19, 1e-30])
def test_tiny_coordinates_float(tpo, O, dev, scale):
    g = torch.Generator().manual_seed(3)
    p1 = torch.randn(2, 1500, 3, generator=g) * scale
    p2 = torch.randn(2, 1300, 3, generator=g) * scale
    check_vs_oracle(O, dev, p1, p2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_huge_coordinates(tpo, O, dev, dtype):
    g = torch.Generator().manual_seed(4)
    p1 = torch.randn(3, 700, 3, generator=g, dtype=torch.float64)
    p2 = torch.randn(3, 1100, 3, generator=g, dtype=torch.float64)
    p2[0, 5] = 2.0 ** 61              # beyond the filter's 2^60 bound
    p2[1, 900, 1] = 1e30              # squares overflow in float
    p1[1, 3, 0] = -1e25               # query with huge coordinate
    p1[2, 17] = p2[2, 40] * 2.0 ** 70
    check_vs_oracle(O, dev, p1.to(dtype), p2.to(dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16])
def test_nonfinite_coordinates_follow_reference(tpo, O, dev, dtype):
    g = torch.Generator().manual_seed(5)
    B, N, M = 6, 600, 1500
    p1 = torch.randn(B, N, 3, generator=g)
    p2 = torch.randn(B, M, 3, generator=g)
    inf, nan = float("inf"), float("nan")
    p2[0, 0, 1] = nan                 # D(0) NaN: every query of batch 0 -> (NaN, 0)
    p2[1, 512, 0] = nan               # stage head: refs 512..1023 never count
    p2[1, 800] = p1[1, 7]             # ... including the exact match of query 7
    p2[2, 700, 2] = nan               # non-head NaN: only ref 700 drops out
    p2[3, 300, 0] = inf               # inf reference
    p2[3, 301, 0] = -inf
    p1[4, 9, 2] = nan                 # NaN query
    p1[4, 10, 0] = inf                # inf query: inf - inf with p2[4, 0]
    p2[4, 0, 0] = inf
    p1[5, :, :] = inf                 # every distance inf or NaN
    i1, i2 = check_vs_oracle(O, dev, p1.to(dtype), p2.to(dtype))
    assert (i1[0] == 0).all() and not np.isin(i1[1], np.arange(512, 1024)).any()


# ---- the spatially pruned float path (both clouds >= 2048 points)

def _pruned_case(kind, g):
    if kind == "uniform":
        return torch.rand(2, 3000, 3, generator=g), torch.rand(2, 2500, 3, generator=g)
    if kind == "blobs":
        return workloads.chamfer_c2(seed=9, B=2, N=4096)
    if kind == "flat":  # zero extent along z: every point in one cell layer
        p1 = torch.rand(2, 2100, 3, generator=g)
        p2 = torch.rand(2, 2600, 3, generator=g)
        p1[..., 2] = 0.5
        p2[..., 2] = 0.5
        return p1, p2
    if kind == "single_point":  # zero extent in every axis, all distances tie
        return torch.full((1, 2048, 3), 0.25), torch.full((1, 2100, 3), 0.75)
    if kind == "apart":  # query cloud far from the reference cloud
        return torch.rand(2, 2500, 3, generator=g) + 10.0, torch.rand(2, 3100, 3, generator=g)
    if kind == "duplicates":
        p1 = torch.rand(2, 2048, 3, generator=g)
        p2 = torch.cat([p1[:, :1024], p1[:, :1024], p1[:, 1000:1100]], 1)[:, torch.randperm(2148, generator=g)]
        return p1, p2
    if kind == "lattice":
        ax = torch.arange(16.0)
        lat = torch.stack(torch.meshgrid(ax, ax, ax, indexing="ij"), -1).reshape(1, -1, 3)
        p2 = lat[:, torch.randperm(lat.shape[1], generator=g)]
        p1 = torch.randint(0, 31, (1, 3000, 3), generator=g).float() / 2
        return p1, p2
    if kind == "line":
        t = torch.rand(1, 4000, 1, generator=g)
        return t * torch.tensor([1.0, 2.0, -1.0]), torch.rand(1, 2500, 1, generator=g) * torch.tensor([1.0, 2.0, -1.0])
    if kind == "tiny":
        return torch.randn(1, 2500, 3, generator=g) * 1e-19, torch.randn(1, 2200, 3, generator=g) * 1e-19
    if kind == "offset":
        return torch.rand(1, 2500, 3, generator=g) + 3e4, torch.rand(1, 2200, 3, generator=g) + 3e4
    if kind == "huge":
        p1, p2 = torch.randn(2, 2300, 3, generator=g), torch.randn(2, 2400, 3, generator=g)
        p2[0, 77] = 2.0 ** 62
        p1[1, 5, 1] = -1e30
        return p1, p2
    if kind == "half_subnormal":  # squared differences below half's normal range
        return (torch.randn(2, 2500, 3, generator=g) * 3e-3,
                torch.randn(2, 2300, 3, generator=g) * 3e-3)
    if kind == "half_overflow":  # far pairs overflow to inf in half; near ones do not
        return (torch.randn(2, 2400, 3, generator=g) * 150,
                torch.randn(2, 2600, 3, generator=g) * 150)
    if kind == "half_all_inf":  # every distance inf in half: ties everywhere
        return (torch.rand(1, 2100, 3, generator=g) + 300.0,
                torch.rand(1, 2200, 3, generator=g) - 300.0)
    if kind == "outlier":  # one far point per cloud: both grids degenerate (dense kernel)
        p1, p2 = workloads.chamfer_c2(seed=10, B=2, N=4096)
        p1[:, 17] = 1e3
        p2[:, 2000] = 1e3
        return p1, p2
    if kind == "outlier_query":  # only the query cloud: far queries scan the whole cloud
        p1, p2 = workloads.chamfer_c2(seed=11, B=2, N=4096)
        p1[0, 17] = 1e3
        p1[1, 5:9] = torch.tensor([-50.0, 80.0, 3.0])
        return p1, p2
    if kind == "heavy_tail":  # far points on several axes and sides: the box is cut
        p1, p2 = workloads.chamfer_c2(seed=12, B=2, N=3000)
        p1[0, :5] = torch.tensor([[1e2, 0, 0], [0, -1e3, 0], [0, 0, 1e4], [-3e2, 2e2, 0], [5e3, 5e3, 5e3]])
        p2[0, 10:13] = torch.tensor([[-1e4, 0, 0], [0, 7e2, 0], [0, 0, -2e3]])
        p1[1, 100] = torch.tensor([0.0, 0.0, -1e5])
        p2[1, 7] = torch.tensor([1e5, 0.0, 0.0])
        return p1, p2
    if kind == "cut_flat":  # a flat cloud plus a few points off the plane
        p1 = torch.rand(2, 2500, 3, generator=g)
        p2 = torch.rand(2, 2300, 3, generator=g)
        p1[..., 2] = 0.5
        p2[..., 2] = 0.5
        p1[:, :2, 2] = torch.tensor([900.0, -700.0])
        p2[:, 5, 2] = 1e3
        return p1, p2
    if kind == "far_clusters":  # two tight clusters far apart: one cell each
        p1 = torch.rand(2, 3000, 3, generator=g) * 0.01
        p2 = torch.rand(2, 2600, 3, generator=g) * 0.01
        p1[:, ::2] += 1e4
        p2[:, 1::3] += 1e4
        return p1, p2
    if kind == "sparse_tail":  # dense core plus a sparse halo: empty rings, big boxes
        p1 = torch.randn(2, 3000, 3, generator=g) * 0.02
        p2 = torch.randn(2, 2500, 3, generator=g) * 0.02
        p1[:, :100] = torch.randn(2, 100, 3, generator=g) * 5
        p2[:, :60] = torch.randn(2, 60, 3, generator=g) * 5
        return p1, p2
    if kind == "nonfinite":
        p1, p2 = torch.randn(3, 2100, 3, generator=g), torch.randn(3, 2600, 3, generator=g)
        p2[0, 1000, 0] = float("nan")   # reference cloud with a NaN: every query re-scanned
        p2[1, 0, 2] = float("nan")      # D(0) NaN
        p1[2, 7, 1] = float("inf")      # one query non-finite
        return p1, p2
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["uniform", "blobs", "flat", "single_point", "apart",
                                  "duplicates", "lattice", "line", "tiny", "offset", "huge",
                                  "outlier", "outlier_query", "heavy_tail", "cut_flat",
                                  "far_clusters", "sparse_tail",
                                  "nonfinite"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_pruned_forward_vs_oracle(tpo, O, dev, kind, dtype):
    g = torch.Generator().manual_seed(len(kind))
    p1, p2 = _pruned_case(kind, g)
    assert min(p1.shape[1], p2.shape[1]) >= 2048
    check_vs_oracle(O, dev, p1.to(dtype), p2.to(dtype))


@pytest.mark.parametrize("kind", ["half_subnormal", "half_overflow", "half_all_inf"])
def test_pruned_half_rounding_cases_vs_oracle(tpo, O, dev, kind):
    # the half search prunes with margins for half rounding, subnormal
    # intermediates and overflow to inf
    g = torch.Generator().manual_seed(len(kind))
    p1, p2 = _pruned_case(kind, g)
    check_vs_oracle(O, dev, p1.half(), p2.half())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_pruned_equals_dense_and_counts_pairs(tpo, dev, dtype):
    import ctypes
    from torch_point_ops import _native

    lib = ctypes.CDLL(_native.HIP_LIB)
    P, I = ctypes.c_void_p, ctypes.c_int64
    lib.tpo_chamfer_fwd.argtypes = [ctypes.c_int, P, P, I, I, I, P, P, P, P, P, I, P]
    lib.tpo_chamfer_workspace_size.argtypes = [ctypes.c_int, I, I, I]
    lib.tpo_chamfer_workspace_size.restype = I
    lib.tpo_chamfer_pairs_evaluated.argtypes = [ctypes.c_int, P, I, I, I, P, P]
    p1, p2 = (t.to(dev) for t in workloads.chamfer_c2(dtype=dtype))
    code = 0 if dtype == torch.float32 else 2
    B, N, M = p1.shape[0], p1.shape[1], p2.shape[1]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    outs = []
    ws = torch.empty(lib.tpo_chamfer_workspace_size(code, B, N, M), dtype=torch.uint8,
                     device=dev)
    for w in (None, ws):
        d1 = torch.empty(B, N, device=dev, dtype=dtype)
        d2 = torch.empty(B, M, device=dev, dtype=dtype)
        i1 = torch.empty(B, N, dtype=torch.int32, device=dev)
        i2 = torch.empty(B, M, dtype=torch.int32, device=dev)
        rc = lib.tpo_chamfer_fwd(code, p1.data_ptr(), p2.data_ptr(), B, N, M, d1.data_ptr(),
                                 d2.data_ptr(), i1.data_ptr(), i2.data_ptr(),
                                 None if w is None else w.data_ptr(),
                                 0 if w is None else w.numel(), stream)
        assert rc == 0
        outs.append((d1, d2, i1, i2))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    pairs = torch.zeros(1, dtype=torch.int64, device=dev)
    assert lib.tpo_chamfer_pairs_evaluated(code, ws.data_ptr(), B, N, M, pairs.data_ptr(),
                                           stream) == 0
    n = int(pairs.item())
    assert 0 < n < 2 * B * N * M


# ---- the reference test suite's checks (tests/test_chamfer.py) ----

def torch_reference(p1, p2):
    dm = ((p1.unsqueeze(2) - p2.unsqueeze(1)) ** 2).sum(3)
    return dm.min(2).values, dm.min(1).values


def test_reference_forward_and_known_values(tpo, dev):
    g = torch.Generator().manual_seed(0)
    p1 = torch.randn(1, 64, 3, generator=g).to(dev)
    p2 = torch.randn(1, 128, 3, generator=g).to(dev)
    d1, d2, _, _ = torch.ops.torch_point_ops_chamfer.chamfer_forward(p1, p2)
    r1, r2 = torch_reference(p1, p2)
    assert torch.allclose(d1, r1) and torch.allclose(d2, r2)
    p = torch.tensor([[[0.0, 0.0, 0.0], [1.0, 1.0, 1.0]]], device=dev)
    d1, d2, _, _ = torch.ops.torch_point_ops_chamfer.chamfer_forward(p, p.clone())
    assert (d1 == 0).all() and (d2 == 0).all()
    d1, d2, _, _ = torch.ops.torch_point_ops_chamfer.chamfer_forward(
        torch.zeros(1, 1, 3, device=dev), torch.tensor([[[1.0, 2.0, 3.0]]], device=dev))
    assert d1.item() == 14.0 and d2.item() == 14.0


def test_empty_clouds(tpo, dev):
    p1 = torch.randn(2, 10, 3, device=dev)
    e = torch.empty(2, 0, 3, device=dev)
    d1, d2, i1, i2 = torch.ops.torch_point_ops_chamfer.chamfer_forward(p1, e)
    assert d1.shape == (2, 10) and d2.shape == (2, 0)
    assert (d1 == 0).all() and (i1 == 0).all()
    d1, d2, _, _ = torch.ops.torch_point_ops_chamfer.chamfer_forward(e, p1)
    assert d1.shape == (2, 0) and d2.shape == (2, 10)
    d1, d2, _, _ = torch.ops.torch_point_ops_chamfer.chamfer_forward(e, e)
    assert d1.shape == (2, 0) and d2.shape == (2, 0)


@pytest.mark.parametrize("B,N,M", [(1, 3, 4), (2, 5, 7), (1, 8, 6), (2, 6, 8), (1, 64, 128)])
def test_gradients_vs_torch_reference(tpo, dev, B, N, M):
    g = torch.Generator().manual_seed(N * M)
    p1 = torch.randn(B, N, 3, generator=g).to(dev).requires_grad_(True)
    p2 = torch.randn(B, M, 3, generator=g).to(dev).requires_grad_(True)
    d1, d2 = tpo.chamfer_distance(p1, p2)
    loss = d1.mean() + d2.mean()
    ga, gb = torch.autograd.grad(loss, (p1, p2))
    r1, r2 = torch_reference(p1, p2)
    ref_loss = r1.mean() + r2.mean()
    ra, rb = torch.autograd.grad(ref_loss, (p1, p2))
    assert torch.allclose(loss, ref_loss, atol=1e-6)
    assert torch.allclose(ga, ra, atol=1e-4) and torch.allclose(gb, rb, atol=1e-4)


@pytest.mark.parametrize("which", [1, 2])
def test_gradient_through_one_output(tpo, dev, which):
    # the other distance output (and both index outputs) get no gradient
    g = torch.Generator().manual_seed(40 + which)
    p1 = torch.randn(2, 37, 3, generator=g).to(dev).requires_grad_(True)
    p2 = torch.randn(2, 29, 3, generator=g).to(dev).requires_grad_(True)
    d1, d2 = tpo.chamfer_distance(p1, p2)
    ga, gb = torch.autograd.grad((d1 if which == 1 else d2).sum(), (p1, p2))
    r1, r2 = torch_reference(p1, p2)
    ra, rb = torch.autograd.grad((r1 if which == 1 else r2).sum(), (p1, p2))
    assert torch.allclose(ga, ra, atol=1e-4) and torch.allclose(gb, rb, atol=1e-4)


@pytest.mark.parametrize("red", ["mean", "sum"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16])
@pytest.mark.parametrize("shape", [(2, 37, 29), (3, 3000, 2500), (1, 0, 5), (0, 4, 4)])
def test_module_loss_matches_unfused_reduction(tpo, dev, red, dtype, shape):
    # ChamferDistance(reduction) reduces inside the kernels; the reference
    # module reduces chamfer_forward's distances with torch (chamfer.py:18-24)
    B, N, M = shape
    g = torch.Generator().manual_seed(50 + N)
    p1 = torch.randn(B, N, 3, generator=g).to(dev, dtype)
    p2 = (torch.randn(B, M, 3, generator=g) * 1.5).to(dev, dtype)
    a, b = p1.clone().requires_grad_(True), p2.clone().requires_grad_(True)
    loss = tpo.ChamferDistance(red)(a, b)
    d1, d2 = tpo.chamfer_distance(p1, p2)
    ref = d1.mean() + d2.mean() if red == "mean" else d1.sum() + d2.sum()
    assert loss.dtype == dtype and loss.shape == ()
    rtol = {torch.float32: 1e-5, torch.float64: 1e-12, torch.float16: 2e-3}[dtype]
    assert torch.allclose(loss, ref, rtol=rtol, atol=0, equal_nan=True), (loss, ref)
    assert torch.equal(loss, tpo.ChamferDistance(red)(p1, p2)) or torch.isnan(loss)
    if B * (N + M) == 0:
        return
    ga, gb = torch.autograd.grad(loss, (a, b))
    a2, b2 = p1.clone().requires_grad_(True), p2.clone().requires_grad_(True)
    e1, e2 = tpo.chamfer_distance(a2, b2)
    r = e1.mean() + e2.mean() if red == "mean" else e1.sum() + e2.sum()
    ra, rb = torch.autograd.grad(r, (a2, b2))
    # same per-point gradient, same kernel: equal up to the order of atomic sums
    gtol = 1e-2 if dtype == torch.float16 else 1e-6
    for got, want in ((ga, ra), (gb, rb)):
        assert got.shape == want.shape
        if want.numel() == 0:
            continue
        scale = max(want.abs().max().item(), 1e-30)
        assert (got - want).abs().max().item() <= gtol * scale


def test_module_loss_at_headline_size(tpo, dev):
    # many search workgroups on every XCD feed the last-workgroup reduction
    p1, p2 = (t.to(dev) for t in workloads.chamfer_c2(B=8))
    loss = tpo.ChamferDistance("mean")(p1, p2)
    d1, d2 = tpo.chamfer_distance(p1, p2)
    e1 = d1.double().mean() + d2.double().mean()
    assert abs(loss.item() - e1.item()) <= 1e-5 * abs(e1.item())
    for _ in range(3):
        assert torch.equal(loss, tpo.ChamferDistance("mean")(p1, p2))


def test_gradcheck_float64(tpo, dev):
    g = torch.Generator().manual_seed(5)
    p1 = torch.randn(1, 4, 3, generator=g, dtype=torch.float64).to(dev).requires_grad_(True)
    p2 = torch.randn(1, 5, 3, generator=g, dtype=torch.float64).to(dev).requires_grad_(True)
    assert torch.autograd.gradcheck(tpo.chamfer_distance, (p1, p2), eps=1e-6, atol=1e-5,
                                    rtol=1e-4, nondet_tol=1e-5, fast_mode=True,
                                    check_batched_grad=False)
    model = tpo.ChamferDistance(reduction="mean")
    q1 = p1[:, :3].detach().clone().requires_grad_(True)
    q2 = p2[:, :4].detach().clone().requires_grad_(True)
    assert torch.autograd.gradcheck(model, (q1, q2), eps=1e-6, atol=1e-5, rtol=1e-4,
                                    nondet_tol=1e-5, fast_mode=True, check_batched_grad=False)


def test_opcheck_and_compile(tpo, dev):
    from torch.library import opcheck

    g = torch.Generator().manual_seed(6)
    p1 = torch.randn(1, 3, 3, generator=g).to(dev)
    p2 = torch.randn(1, 3, 3, generator=g).to(dev)
    opcheck(torch.ops.torch_point_ops_chamfer.chamfer_forward.default, (p1, p2),
            raise_exception=True)
    for mean in (True, False):
        opcheck(torch.ops.torch_point_ops_chamfer.chamfer_loss_forward.default,
                (p1.clone().requires_grad_(True), p2.clone().requires_grad_(True), mean),
                raise_exception=True)
    model = tpo.ChamferDistance().to(dev)
    a = torch.randn(1, 64, 3, generator=g).to(dev)
    b = torch.randn(1, 128, 3, generator=g).to(dev)
    assert torch.equal(model(a, b), torch.compile(model)(a, b))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.float64])
def test_multi_precision_and_reductions(tpo, dev, dtype):
    g = torch.Generator().manual_seed(7)
    p1 = torch.randn(2, 10, 3, generator=g).to(dev, dtype)
    p2 = torch.randn(2, 12, 3, generator=g).to(dev, dtype)
    d1, d2 = tpo.chamfer_distance(p1, p2)
    assert d1.dtype == dtype and d1.shape == (2, 10) and d2.shape == (2, 12)
    a, b = p1.clone().requires_grad_(True), p2.clone().requires_grad_(True)
    e1, e2 = tpo.chamfer_distance(a, b)
    (e1.mean() + e2.mean()).backward()
    assert torch.isfinite(a.grad).all() and torch.isfinite(b.grad).all()
    for red in ("mean", "sum", None, "none"):
        r = tpo.ChamferDistance(reduction=red)(p1, p2)
        if red in (None, "none"):
            assert len(r) == 2 and r[0].dtype == dtype
        else:
            assert r.dtype == dtype


def test_non_contiguous_inputs(tpo, O, dev):
    g = torch.Generator().manual_seed(8)
    base = torch.randn(2, 3, 50, generator=g)
    p1 = base.transpose(1, 2)  # (2, 50, 3) non-contiguous
    p2 = torch.randn(2, 40, 3, generator=g)
    d1, d2 = tpo.chamfer_distance(p1.to(dev), p2.to(dev))
    e1, e2, _, _ = O.chamfer_fwd(np_(p1.contiguous()), np_(p2))
    assert_bits(np_(d1), e1)
    assert_bits(np_(d2), e2)
