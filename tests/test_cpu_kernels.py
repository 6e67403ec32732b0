"""The CPU dispatch-key kernels (csrc/cpu_ops.cpp) against the oracle's
restatement of the reference's CPU kernels (knn.cpp:30-164, fps.cpp:18-155),
bit for bit, plus the reference tests' CPU-side checks (gradcheck on float64,
the CPU fallback tests of tests/test_fps.py:358-372 and :701-717)."""
import numpy as np
import pytest
import torch

DTYPES = [torch.float32, torch.float64, torch.float16]

pytestmark = pytest.mark.usefixtures("tpo")  # registers the operators


def bits(t):
    a = t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else t
    return a.view(np.uint8)


def knn_inputs(seed, dt, N=4, P1=300, P2=400, D=3, lattice=False):
    g = torch.Generator().manual_seed(seed)
    if lattice:
        p1 = torch.randint(-3, 4, (N, P1, D), generator=g).to(dt)
        p2 = torch.randint(-3, 4, (N, P2, D), generator=g).to(dt)
    else:
        p1 = torch.randn(N, P1, D, generator=g).to(dt)
        p2 = torch.randn(N, P2, D, generator=g).to(dt)
    l1 = torch.randint(P1 // 2, P1 + 1, (N,), generator=g)
    l2 = torch.randint(1, P2 + 1, (N,), generator=g)
    l2[0] = 3  # fewer references than K: padding
    return p1, p2, l1, l2


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("norm", [1, 2])
@pytest.mark.parametrize("K,D,lattice", [(1, 3, False), (5, 3, True), (16, 3, False),
                                         (40, 7, False), (8, 64, False)])
def test_knn_cpu_forward_backward_vs_oracle(O, dt, norm, K, D, lattice):
    p1, p2, l1, l2 = knn_inputs(K * 10 + D, dt, D=D, lattice=lattice)
    idx, d = torch.ops.torch_point_ops_knn.knn_forward(p1, p2, l1, l2, norm, K, -1)
    ei, ed = O.cpu_knn_fwd(p1.numpy(), p2.numpy(), l1.numpy(), l2.numpy(), K, norm)
    assert idx.dtype == torch.int64 and d.dtype == dt
    assert np.array_equal(idx.numpy(), ei)
    assert np.array_equal(bits(d), bits(ed))
    g = torch.randn(idx.shape, generator=torch.Generator().manual_seed(7)).to(dt)
    g1, g2 = torch.ops.torch_point_ops_knn.knn_backward(p1, p2, l1, l2, idx, norm, g)
    e1, e2 = O.cpu_knn_bwd(p1.numpy(), p2.numpy(), l1.numpy(), l2.numpy(), idx.numpy(), norm,
                           g.numpy())
    assert np.array_equal(bits(g1), bits(e1))
    assert np.array_equal(bits(g2), bits(e2))


def test_knn_cpu_edge_cases(O):
    p1, p2, l1, l2 = knn_inputs(3, torch.float32, N=3, P1=20, P2=30)
    # lengths past the cloud are clamped, negative lengths mean empty
    l1 = torch.tensor([25, 0, -4])
    l2 = torch.tensor([40, 30, 30])
    idx, d = torch.ops.torch_point_ops_knn.knn_forward(p1, p2, l1, l2, 2, 4, -1)
    ei, ed = O.cpu_knn_fwd(p1.numpy(), p2.numpy(), l1.numpy(), l2.numpy(), 4, 2)
    assert np.array_equal(idx.numpy(), ei) and np.array_equal(bits(d), bits(ed))
    assert (idx[1:] == -1).all() and (d[1:] == 0).all()
    # K = 0 and empty clouds
    i0, d0 = torch.ops.torch_point_ops_knn.knn_forward(p1, p2, l1, l2, 2, 0, -1)
    assert i0.shape == (3, 20, 0) and d0.shape == (3, 20, 0)
    e = torch.zeros(2, 0, 3)
    ie, de = torch.ops.torch_point_ops_knn.knn_forward(e, p2[:2], torch.zeros(2, dtype=torch.long),
                                                       torch.full((2,), 30), 2, 3, -1)
    assert ie.shape == (2, 0, 3)
    with pytest.raises(RuntimeError, match="BFloat16"):
        torch.ops.torch_point_ops_knn.knn_forward(p1.bfloat16(), p2.bfloat16(), l1, l2, 2, 4, -1)
    with pytest.raises(RuntimeError, match="Norm must be 1 or 2"):
        torch.ops.torch_point_ops_knn.knn_forward(p1, p2, l1, l2, 3, 4, -1)


def test_knn_cpu_gradcheck():
    """tests/test_knn.py:136-158 of the reference, on this build's CPU kernel."""
    import torch_point_ops as tpo

    g = torch.Generator().manual_seed(5)
    p1 = torch.randn(1, 4, 3, generator=g, dtype=torch.float64, requires_grad=True)
    p2 = torch.randn(1, 5, 3, generator=g, dtype=torch.float64, requires_grad=True)
    for norm in (1, 2):
        def f(a, b):
            return tpo.knn_points(a, b, K=2, norm=norm, return_sorted=False)[1].sum()

        assert torch.autograd.gradcheck(f, (p1, p2), eps=1e-6, atol=1e-5, rtol=1e-4)

        def fs(a, b):
            return tpo.knn_points(a, b, K=3, norm=norm)[1].mean()

        assert torch.autograd.gradcheck(fs, (p1, p2), eps=1e-6, atol=1e-5, rtol=1e-4)


def test_knn_points_module_on_cpu(O):
    """knn_points / KNearestNeighbors / knn_gather on host tensors go through
    the CPU kernel and the reference's Python post-processing."""
    import torch_point_ops as tpo

    p1, p2, l1, l2 = knn_inputs(11, torch.float32, N=3, P1=50, P2=60)
    idx, d = tpo.knn_points(p1, p2, l1, l2, K=6)
    ei, ed = O.cpu_knn_fwd(p1.numpy(), p2.numpy(), l1.numpy(), l2.numpy(), 6, 2)
    # the CPU kernel's rows are already ascending with distinct values here;
    # the wrapper's sort keeps them, padding (dist 0) is reported as 0
    assert np.array_equal(d.numpy(), ed)
    valid = ed > 0
    assert np.array_equal(idx.numpy()[valid], ei[valid])
    # return_nn gathers with the reference's torch ops, which (like the
    # reference) reject the CPU kernel's -1 padding: use full lengths here
    l1, l2 = torch.full((3,), 50), torch.full((3,), 60)
    idx, d = tpo.knn_points(p1, p2, l1, l2, K=6)
    m = tpo.KNearestNeighbors(K=6, return_nn=True)
    out = m(p1, p2, l1, l2)
    assert torch.equal(out[0], idx) and torch.equal(out[1], d)
    nn = out[2]
    assert nn.shape == (3, 50, 6, 3)
    j = idx[1, 4, 2]
    assert torch.equal(nn[1, 4, 2], p2[1, j])


@pytest.mark.parametrize("dt", DTYPES)
def test_fps_cpu_vs_oracle(O, dt):
    g = torch.Generator().manual_seed(21)
    pts = torch.randn(5, 400, 3, generator=g).to(dt)
    pts[1] = torch.randint(-2, 3, (400, 3), generator=g).to(dt)  # lattice ties
    pts[2, 10:14] = 0.0  # degenerate points: chosen first on the CPU path
    s = torch.ops.torch_point_ops_fps.fps_forward(pts, 64)
    assert s.dtype == torch.int64
    assert np.array_equal(s.numpy(), O.cpu_fps(pts.numpy(), 64))
    assert s[2, 1:5].tolist() == [10, 11, 12, 13]


def test_fps_cpu_large_cloud_chunked(O):
    """One big cloud: the kernel splits the points over threads per sample."""
    g = torch.Generator().manual_seed(22)
    pts = torch.rand(1, 20000, 3, generator=g) * 2 - 1
    pts[0, 5000:5100] = torch.randint(-1, 2, (100, 3), generator=g).float()  # ties
    s = torch.ops.torch_point_ops_fps.fps_forward(pts, 257)
    assert np.array_equal(s.numpy(), O.cpu_fps(pts.numpy(), 257))
    q = torch.ops.torch_point_ops_quick_fps.quick_fps_forward(pts, 257, 6)
    assert torch.equal(q, s)


def test_fps_cpu_fallback_reference_tests():
    """tests/test_fps.py:358-372 and :701-717 of the reference."""
    import torch_point_ops as tpo

    points = torch.randn(1, 15, 3)
    indices = tpo.furthest_point_sampling(points, 5)
    assert indices.shape == (1, 5) and indices.device.type == "cpu"
    features = torch.randn(1, 4, 15)
    gathered = tpo.gather_points(features, indices)
    assert gathered.shape == (1, 4, 5) and gathered.device.type == "cpu"
    points = torch.randn(1, 30, 3)
    for kd in (3, 4, 5, 6):
        q = tpo.quick_furthest_point_sampling(points, 8, kd)
        assert q.shape == (1, 8) and len(torch.unique(q[0])) == 8
    fps_mod = tpo.FarthestPointSampling(6)
    idx = fps_mod(points)
    assert torch.equal(idx, tpo.furthest_point_sampling(points, 6))
    with pytest.raises(RuntimeError, match="kd_depth must be between 1 and 10"):
        torch.ops.torch_point_ops_quick_fps.quick_fps_forward(points, 8, 11)
    with pytest.raises(RuntimeError, match="cannot exceed number of points"):
        torch.ops.torch_point_ops_fps.fps_forward(points, 31)


@pytest.mark.parametrize("dt", DTYPES)
def test_gather_cpu_vs_oracle(O, dt):
    g = torch.Generator().manual_seed(23)
    f = torch.randn(3, 7, 90, generator=g).to(dt)
    idx = torch.randint(0, 90, (3, 130), generator=g)  # duplicates
    out = torch.ops.torch_point_ops_fps.gather_points_forward(f, idx)
    assert np.array_equal(bits(out), bits(O.cpu_gather_fwd(f.numpy(), idx.numpy())))
    go = torch.randn(3, 7, 130, generator=g).to(dt)
    gb = torch.ops.torch_point_ops_fps.gather_points_backward(go, idx, 90)
    assert np.array_equal(bits(gb), bits(O.cpu_gather_bwd(go.numpy(), idx.numpy(), 90)))


def test_gather_cpu_gradcheck():
    """tests/test_fps.py:374-396 of the reference, on the CPU kernels."""
    import torch_point_ops as tpo

    points = torch.randn(1, 3, 5, dtype=torch.float64, requires_grad=True)
    idx = torch.tensor([[0, 2, 4, 2]])
    assert torch.autograd.gradcheck(lambda p: tpo.gather_points(p, idx).sum(), (points,),
                                    eps=1e-6, atol=1e-5, rtol=1e-4)
