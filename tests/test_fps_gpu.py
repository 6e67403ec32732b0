"""FPS and gather_points on the GPU vs the oracle (indices identical) and the
reference test suite's semantics (tests/test_fps.py)."""
import numpy as np
import pytest
import torch

import workloads

pytestmark = pytest.mark.gpu


def np_(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16])
@pytest.mark.parametrize("B,N,m", [(1, 1, 1), (2, 5, 5), (2, 20, 5), (3, 100, 30),
                                   (2, 1000, 200), (1, 4097, 500), (2, 65536, 64)])
def test_fps_vs_oracle(tpo, O, dev, dtype, B, N, m):
    g = torch.Generator().manual_seed(N + m)
    pts = torch.randn(B, N, 3, generator=g).to(dtype)
    got = tpo.furthest_point_sampling(pts.to(dev), m)
    assert np.array_equal(np_(got), O.fps(np_(pts), m))


def test_fps_degenerate_and_ties(tpo, O, dev):
    g = torch.Generator().manual_seed(3)
    cases = [
        torch.randn(1, 20, 3, generator=g) * 1e-6,                  # all skipped -> zeros
        torch.randint(-2, 3, (2, 300, 3), generator=g).float(),      # integer grid: many ties
        torch.randint(-1, 2, (1, 5000, 3), generator=g).float() * 0.5,
    ]
    p = torch.randn(1, 10, 3, generator=g)
    p[0, 5:8] = 1e-4
    cases.append(p)
    ang = torch.arange(1023, dtype=torch.float64) * (2 * np.pi / 1023)
    circ = torch.stack([ang.cos(), ang.sin(), torch.zeros_like(ang)], 1)
    cases.append(torch.cat([torch.zeros(1, 3, dtype=torch.float64), circ]).float()[None])
    cases.append(torch.randn(1, 20, 3, generator=g) * 1e6)         # temp saturates at 1e10
    for pts in cases:
        m = min(pts.shape[1], 40)
        got = tpo.furthest_point_sampling(pts.to(dev), m)
        assert np.array_equal(np_(got), O.fps(np_(pts), m))
    assert (np_(tpo.furthest_point_sampling(cases[0].to(dev), 8)) == 0).all()


def test_fps_large_n_bucket_path(tpo, O, dev):
    """N > 65536 uses buckets of more than 64 points."""
    g = torch.Generator().manual_seed(4)
    pts = torch.rand(1, 70001, 3, generator=g) * 2 - 1
    got = tpo.furthest_point_sampling(pts.to(dev), 100)
    assert np.array_equal(np_(got), O.fps(np_(pts), 100))


def test_quick_fps_equals_fps(tpo, O, dev):
    """quick_fps_forward is served by the exact kernel: the reference suite
    asserts quick == regular FPS on exact inputs (tests/test_fps.py:1128-1291);
    here both are compared with the oracle, on a cloud large enough for the
    bucket-pruned path, for every kd_depth class."""
    g = torch.Generator().manual_seed(5)
    for pts in (torch.randn(2, 500, 3, generator=g), torch.rand(2, 20000, 3, generator=g) * 2 - 1):
        ref = O.fps(np_(pts), 300)
        a = tpo.furthest_point_sampling(pts.to(dev), 300)
        assert np.array_equal(np_(a), ref)
        for d in (1, 3, 4, 6, 10):
            q = tpo.quick_furthest_point_sampling(pts.to(dev), 300, kd_depth=d)
            assert np.array_equal(np_(q), ref)
            assert np.array_equal(np_(torch.ops.torch_point_ops_quick_fps.quick_fps_forward(
                pts.to(dev), 300, d)), ref)
    pts = pts.to(dev)
    i, s = tpo.quick_farthest_point_sample_and_gather(pts, 20, kd_depth=5)
    assert torch.equal(s, pts[torch.arange(2, device=dev)[:, None], i])


# ------------------------------------------------------------------- gather

@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16])
def test_gather_vs_oracle(tpo, O, dev, dtype):
    g = torch.Generator().manual_seed(6)
    pts = torch.randn(3, 13, 777, generator=g).to(dtype)
    idx = torch.randint(0, 777, (3, 130), generator=g)
    out = torch.ops.torch_point_ops_fps.gather_points_forward(pts.to(dev), idx.to(dev))
    assert np.array_equal(np_(out), O.gather_fwd(np_(pts), np_(idx)))
    go = torch.randn(3, 13, 130, generator=g).to(dtype)
    gp = torch.ops.torch_point_ops_fps.gather_points_backward(go.to(dev), idx.to(dev), 777)
    ref = O.gather_bwd(np_(go), np_(idx), 777, accum_f64=True)
    tol = 1e-2 if dtype == torch.float16 else 1e-6
    assert np.abs(np_(gp).astype(np.float64) - ref).max() <= tol * np.abs(ref).max()
    # unique indices: every value is exactly 0 + g, bit for bit (a gradient
    # of -0.0 lands as +0.0, as the reference's atomicAdd into zeros leaves it)
    uidx = torch.stack([torch.randperm(777, generator=g)[:130] for _ in range(3)])
    go[:, :, ::7] = -0.0
    gp = torch.ops.torch_point_ops_fps.gather_points_backward(go.to(dev), uidx.to(dev), 777)
    want = O.gather_bwd(np_(go), np_(uidx), 777)
    u = np.dtype(f"u{want.dtype.itemsize}")
    assert np.array_equal(np_(gp).view(u), want.view(u))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16])
@pytest.mark.parametrize("C,N,M", [(1, 3000, 900), (3, 5000, 2000), (5, 9001, 4100),
                                   (64, 4000, 300), (2, 20001, 4096), (2, 40000, 20000)])
def test_gather_backward_paths(tpo, O, dev, dtype, C, N, M):
    """The backward's channel blocks of 1 to 16 rows staged in LDS (the parts
    of one block split the positions), with the position map built in LDS a
    chunk of 8192 positions at a time (M <= 4096; N = 20001: parts of 10000
    and 10001 positions, a full chunk and a ragged one) or in global memory
    (M = 4100), and rows too long for LDS (M = 20000: the dense pass), with
    repeated indices (added by atomics) and without (bit for bit, -0
    gradients landing as +0)."""
    g = torch.Generator().manual_seed(C * 7 + M)
    B = 2
    go = torch.randn(B, C, M, generator=g).to(dtype)
    idx = torch.randint(0, N, (B, M), generator=g)
    idx[:, 1::5] = idx[:, 0::5][:, : idx[:, 1::5].shape[1]]  # every fifth sample repeats
    gp = torch.ops.torch_point_ops_fps.gather_points_backward(go.to(dev), idx.to(dev), N)
    ref = O.gather_bwd(np_(go), np_(idx), N, accum_f64=True)
    tol = 1e-2 if dtype == torch.float16 else 1e-6
    assert np.abs(np_(gp).astype(np.float64) - ref).max() <= tol * np.abs(ref).max()
    uidx = torch.stack([torch.randperm(N, generator=g)[:M] for _ in range(B)])
    go[:, :, ::7] = -0.0
    gp = torch.ops.torch_point_ops_fps.gather_points_backward(go.to(dev), uidx.to(dev), N)
    want = O.gather_bwd(np_(go), np_(uidx), N)
    u = np.dtype(f"u{want.dtype.itemsize}")
    assert np.array_equal(np_(gp).view(u), want.view(u))


def test_gather_config4(tpo, O, dev):
    pts = workloads.fps_c4()
    idx = tpo.furthest_point_sampling(pts.to(dev), 4096)
    feats, go = workloads.gather_c4()
    f = feats.to(dev).requires_grad_(True)
    out = tpo.gather_points(f, idx)
    ref = torch.gather(feats, 2, idx.cpu()[:, None, :].expand(-1, 64, -1))
    assert torch.equal(out.cpu(), ref)
    out.backward(go.to(dev))
    exp = torch.zeros_like(feats).scatter_add_(2, idx.cpu()[:, None, :].expand(-1, 64, -1), go)
    assert torch.equal(f.grad.cpu(), exp)


# ---- the reference test suite's checks (tests/test_fps.py) ----

def test_reference_semantics(tpo, dev):
    g = torch.Generator().manual_seed(7)
    pts = torch.randn(2, 20, 3, generator=g).to(dev)
    idx = tpo.furthest_point_sampling(pts, 5)
    assert idx.shape == (2, 5) and (idx[:, 0] == 0).all()
    assert all(len(torch.unique(idx[n])) == 5 for n in range(2))
    p = torch.randn(1, 100, 3, generator=g).to(dev)
    for m in (1, 5, 10, 25, 50):
        i = tpo.furthest_point_sampling(p, m)
        assert i.shape == (1, m) and len(torch.unique(i)) == m
    assert tpo.furthest_point_sampling(p[:, :10], 1)[0, 0].item() == 0
    assert len(torch.unique(tpo.furthest_point_sampling(p[:, :5], 5))) == 5
    feats = torch.randn(2, 4, 10, generator=g).to(dev).requires_grad_(True)
    ind = torch.stack([torch.randperm(10, generator=g)[:5] for _ in range(2)]).to(dev)
    tpo.gather_points(feats, ind).sum().backward()
    for n in range(2):
        for s in range(5):
            assert abs(feats.grad[n, :, ind[n, s]].sum().item() - 4) < 1e-5
    x = torch.linspace(-1, 1, 5)
    xx, yy = torch.meshgrid(x, x, indexing="ij")
    grid = torch.stack([xx.flatten(), yy.flatten(), torch.zeros(25)], -1)[None].to(dev)
    gi = tpo.furthest_point_sampling(grid, 5)
    assert gi[0, 0].item() == 0 and len(torch.unique(gi)) == 5
    i2, s2 = tpo.farthest_point_sample_and_gather(pts, 8)
    assert torch.equal(s2, pts[torch.arange(2, device=dev)[:, None], i2])
    ii, sp = tpo.FarthestPointSampling(10, return_gathered=True)(pts)
    assert sp.shape == (2, 10, 3)


def test_gradcheck_opcheck_compile(tpo, dev):
    from torch.library import opcheck

    fn = lambda p: tpo.gather_points(p, torch.tensor([[0, 2, 4]], device=dev)).sum()  # noqa
    p = torch.randn(1, 3, 5, device=dev, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(fn, (p,), eps=1e-6, atol=1e-5, rtol=1e-4, fast_mode=True)
    pts = torch.randn(1, 10, 3, device=dev)
    feats = torch.randn(1, 4, 10, device=dev)
    ind = torch.tensor([[0, 2, 4, 6]], device=dev)
    opcheck(torch.ops.torch_point_ops_fps.fps_forward.default, (pts, 4), raise_exception=True)
    opcheck(torch.ops.torch_point_ops_fps.gather_points_forward.default, (feats, ind),
            raise_exception=True)
    p = torch.randn(1, 20, 3, device=dev)
    e = tpo.furthest_point_sampling(p, 8)
    c = torch.compile(tpo.furthest_point_sampling)(p, 8)
    assert torch.equal(e, c)
    f = torch.randn(1, 6, 20, device=dev)
    assert torch.allclose(tpo.gather_points(f, e), torch.compile(tpo.gather_points)(f, e))
    for dtype in (torch.float16, torch.float32, torch.float64):
        q = torch.randn(1, 20, 3, device=dev, dtype=dtype)
        i = tpo.furthest_point_sampling(q, 8)
        assert i.dtype == torch.int64
        assert tpo.gather_points(torch.randn(1, 4, 20, device=dev, dtype=dtype), i).dtype == dtype
