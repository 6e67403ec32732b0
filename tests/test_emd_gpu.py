"""Earth mover's distance on the GPU vs the oracle (oracle/tpo_oracle.c, a
restatement of emd.cu:18-303) and the reference test suite's semantics
(tests/test_emd.py).

The reference's exponential is CUDA's and the oracle's is the C library's;
the GPU's is ROCm's, and its sums run in a parallel order.  Parity is
therefore to a tolerance, stated per dtype below:
  float32  cost and match within 1e-4 relative (+ 1e-6 of the mass scale);
  float64  within 1e-6 relative: remain/ratio values pass through float in
           the reference's fminf/fmaxf, so float roundings can differ;
  float16  within 3e-2 relative: ratios and match are stored in half at
           every level, and one half ulp is 1e-3.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _registered(tpo):
    """Importing torch_point_ops registers the torch_point_ops_emd ops."""

# (rtol, atol as a fraction of the largest match entry) per dtype
TOL = {torch.float32: (1e-4, 1e-6), torch.float64: (1e-6, 1e-9), torch.float16: (3e-2, 2e-3)}


def np_(t):
    return t.detach().cpu().numpy()


def clouds(B, n, m, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    p1 = torch.randn(B, n, 3, generator=g, dtype=torch.float64).to(dtype)
    p2 = torch.randn(B, m, 3, generator=g, dtype=torch.float64).to(dtype)
    return p1, p2


def close(a, b, rtol, atol_frac, scale=None):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if scale is None:
        scale = max(np.abs(b).max() if b.size else 0.0, 1e-30)
    err = np.abs(a - b)
    ok = err <= rtol * np.abs(b) + atol_frac * scale
    assert ok.all(), f"max err {err.max():.3g} (scale {scale:.3g}), {np.sum(~ok)} of {a.size} off"


SHAPES = [(2, 128, 128), (2, 64, 128), (2, 128, 64), (1, 1, 1), (2, 1, 5), (2, 5, 1),
          (3, 100, 37), (1, 300, 257)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16])
@pytest.mark.parametrize("shape", SHAPES)
def test_forward_backward_vs_oracle(O, dev, dtype, shape):
    B, n, m = shape
    p1, p2 = clouds(B, n, m, dtype, seed=n * 1000 + m)
    cost, match = torch.ops.torch_point_ops_emd.emd_forward(p1.to(dev), p2.to(dev))
    ec, em = O.emd_fwd(np_(p1), np_(p2))
    assert cost.dtype == dtype and match.shape == (B, m, n)
    rtol, af = TOL[dtype]
    close(np_(match), em, rtol, af)
    close(np_(cost), ec, rtol, af, scale=np.abs(ec).max())
    # backward on the GPU's own match, against the oracle's emd.cu:234-303
    gc = torch.rand(B, generator=torch.Generator().manual_seed(7), dtype=torch.float64).to(dtype)
    g1, g2 = torch.ops.torch_point_ops_emd.emd_backward(gc.to(dev), p1.to(dev), p2.to(dev), match)
    e1, e2 = O.emd_bwd(np_(gc), np_(p1), np_(p2), np_(match))
    grtol = {torch.float32: 1e-4, torch.float64: 1e-9, torch.float16: 2e-2}[dtype]
    close(np_(g1), e1, grtol, grtol, scale=np.abs(e1).max())
    close(np_(g2), e2, grtol, grtol, scale=np.abs(e2).max())


def test_headline_size_cloud_vs_oracle(O, dev):
    """B16 N2048 M2048 (the reference benchmark's size): cloud 0 against the
    oracle, every cloud against the transport-plan properties."""
    p1, p2 = clouds(16, 2048, 2048, torch.float32, seed=3)
    cost, match = torch.ops.torch_point_ops_emd.emd_forward(p1.to(dev), p2.to(dev))
    ec, em = O.emd_fwd(np_(p1[:1]), np_(p2[:1]))
    # sums of 2048 terms in another order: a few plan entries (17 of 4.2M
    # measured) move by up to 1e-4 of the unit mass; the cost by far less
    close(np_(match[:1]), em, 1e-4, 2e-4)
    close(np_(cost[:1]), ec, 1e-4, 0.0)
    mt = match.double()
    assert (mt >= 0).all()
    # every point's mass is 1 here (n == m); no row or column over-spends it
    assert (mt.sum(1) <= 1 + 1e-4).all() and (mt.sum(2) <= 1 + 1e-4).all()
    assert torch.allclose(mt.sum((1, 2)), torch.full((16,), 2048.0, dtype=torch.float64,
                                                     device=dev), rtol=1e-4)


@pytest.mark.parametrize("case", ["kd_largest_with_morton", "morton_with_kd", "far_clusters"])
def test_point_orders_and_far_point_pruning_vs_oracle(O, dev, case):
    """The sweeps hold their own points in runs of 64 listed by a k-d tree
    (clouds of up to 4096 points) or by Morton cells (larger clouds), one
    kind per cloud; at the steep levels they leave out the points of the
    other cloud beyond every level's zero distance from the run's box.
    Neither changes a sum: checked against the oracle on both kinds of cloud
    side by side, and on clusters far apart (scale 100) where most points are
    left out of most sweeps."""
    if case == "kd_largest_with_morton":
        p1, p2 = clouds(1, 4096, 4097, torch.float32, seed=31)
    elif case == "morton_with_kd":
        p1, p2 = clouds(1, 4100, 1500, torch.float32, seed=33)
    else:
        g = torch.Generator().manual_seed(34)
        c = torch.randn(6, 3, generator=g, dtype=torch.float64) * 100
        p1 = (c[torch.randint(0, 6, (2, 1800), generator=g)] +
              torch.randn(2, 1800, 3, generator=g, dtype=torch.float64)).float()
        p2 = (c[torch.randint(0, 6, (2, 1300), generator=g)] +
              torch.randn(2, 1300, 3, generator=g, dtype=torch.float64)).float()
    cost, match = torch.ops.torch_point_ops_emd.emd_forward(p1.to(dev), p2.to(dev))
    ec, em = O.emd_fwd(np_(p1), np_(p2))
    close(np_(match), em, 1e-4, 2e-4)
    close(np_(cost), ec, 1e-4, 0.0, scale=np.abs(ec).max())


def test_deterministic(dev):
    p1, p2 = clouds(4, 500, 700, torch.float32, seed=11)
    a = torch.ops.torch_point_ops_emd.emd_forward(p1.to(dev), p2.to(dev))
    b = torch.ops.torch_point_ops_emd.emd_forward(p1.to(dev), p2.to(dev))
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


# ---- the reference test suite (tests/test_emd.py) ----

def test_forward_shape(tpo, dev):  # test_emd.py:70-78
    p1, p2 = clouds(1, 64, 128, torch.float64, seed=1)
    dist = tpo.earth_movers_distance(p1.to(dev), p2.to(dev))
    assert dist.dim() == 1 and dist.shape[0] == 1


def test_known_values(tpo, dev):  # test_emd.py:151-171
    p = torch.tensor([[[0.0, 0.0, 0.0], [1.0, 1.0, 1.0]]], device=dev)
    assert torch.allclose(tpo.earth_movers_distance(p, p.clone()), torch.zeros(1, device=dev),
                          atol=1e-6)
    q, _ = clouds(2, 128, 128, torch.float64, seed=2)
    q = q.to(dev)
    assert torch.allclose(tpo.earth_movers_distance(q, q), torch.zeros(2, device=dev,
                                                                       dtype=torch.float64),
                          atol=1e-5)


def test_static_values(tpo, dev):  # test_emd.py:173-220
    p1 = torch.tensor([[[1.7, -0.1, 0.1], [0.1, 1.2, 0.3]]], device=dev).repeat(3, 1, 1)
    p2 = torch.tensor([[[0.3, 1.8, 0.2], [1.2, -0.2, 0.3]]], device=dev).repeat(3, 1, 1)
    p1.requires_grad = True
    p2.requires_grad = True
    dist = tpo.earth_movers_distance(p1, p2)
    (dist[0] / 2 + dist[1] * 2 + dist[2] / 3).backward()
    assert torch.allclose(dist, torch.tensor([0.355] * 3, device=dev), atol=1e-3)
    e1 = torch.tensor([[[0.2500, 0.0500, -0.1000], [-0.1000, -0.3000, 0.0500]],
                       [[1.0000, 0.2000, -0.4000], [-0.4000, -1.2000, 0.2000]],
                       [[0.1667, 0.0333, -0.0667], [-0.0667, -0.2000, 0.0333]]], device=dev)
    e2 = torch.tensor([[[0.1000, 0.3000, -0.0500], [-0.2500, -0.0500, 0.1000]],
                       [[0.4000, 1.2000, -0.2000], [-1.0000, -0.2000, 0.4000]],
                       [[0.0667, 0.2000, -0.0333], [-0.1667, -0.0333, 0.0667]]], device=dev)
    assert torch.allclose(p1.grad, e1, atol=1e-4)
    assert torch.allclose(p2.grad, e2, atol=1e-4)


def test_empty_clouds(tpo, dev):  # test_emd.py:222-234
    p1 = torch.randn(2, 10, 3, device=dev)
    pe = torch.empty(2, 0, 3, device=dev)
    for a, b in ((p1, pe), (pe, p1), (pe, pe)):
        assert torch.all(tpo.earth_movers_distance(a, b) == 0)
    cost, match = torch.ops.torch_point_ops_emd.emd_forward(p1, pe)
    assert torch.all(cost == 0) and match.shape == (2, 0, 10)
    a = p1.clone().requires_grad_(True)
    b = torch.empty(2, 0, 3, device=dev, requires_grad=True)
    torch.ops.torch_point_ops_emd.emd_forward(a, b)[0].sum().backward()
    assert torch.all(a.grad == 0) and b.grad.shape == (2, 0, 3)


def test_opcheck(dev):  # test_emd.py:236-253
    from torch.library import opcheck

    p1, p2 = clouds(1, 64, 128, torch.float64, seed=5)
    opcheck(torch.ops.torch_point_ops_emd.emd_forward.default,
            (p1.to(dev).requires_grad_(True), p2.to(dev).requires_grad_(True)),
            raise_exception=True)
    opcheck(torch.ops.torch_point_ops_emd.emd_forward.default, (p1.to(dev), p2.to(dev)),
            raise_exception=True)


def test_compile(tpo, dev):  # test_emd.py:255-264
    model = tpo.EarthMoverDistance().to(dev)
    p1, p2 = clouds(1, 64, 128, torch.float32, seed=6)
    p1, p2 = p1.to(dev), p2.to(dev)
    eager = model(p1, p2)
    compiled = torch.compile(model)(p1, p2)
    assert torch.equal(eager, compiled)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.float64])
def test_multi_precision(tpo, dev, dtype):  # test_emd.py:266-321
    for n, m in ((128, 128), (64, 128)):
        p1, p2 = clouds(2, n, m, dtype, seed=n + m)
        a = p1.to(dev).requires_grad_(True)
        b = p2.to(dev).requires_grad_(True)
        dist = tpo.earth_movers_distance(a, b)
        assert torch.isfinite(dist).all() and (dist >= 0).all() and dist.dtype == dtype
        dist.sum().backward()
        assert torch.isfinite(a.grad).all() and torch.isfinite(b.grad).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.float64])
def test_symmetry(O, tpo, dev, dtype):  # test_emd.py:323-350
    """The swap changes the approximate matching (by up to ~0.08 in cost/n at
    n = 256 in the reference's own algorithm, see the oracle's tests): the
    GPU reproduces the oracle on both orders, and the gap stays bounded."""
    p1, p2 = clouds(2, 256, 256, dtype, seed=9)
    d1 = tpo.earth_movers_distance(p1.to(dev), p2.to(dev))
    d2 = tpo.earth_movers_distance(p2.to(dev), p1.to(dev))
    rtol = TOL[dtype][0]
    close(np_(d1), O.emd_fwd(np_(p1), np_(p2))[0].astype(np.float64) / 256, rtol, rtol)
    close(np_(d2), O.emd_fwd(np_(p2), np_(p1))[0].astype(np.float64) / 256, rtol, rtol)
    assert torch.allclose(d1.double(), d2.double(), atol=0.2)


def test_module_mean_and_gradient(tpo, dev):
    p1, p2 = clouds(3, 200, 150, torch.float32, seed=12)
    a = p1.to(dev).requires_grad_(True)
    b = p2.to(dev).requires_grad_(True)
    loss = tpo.EarthMoverDistance()(a, b)
    loss.backward()
    cost, match = torch.ops.torch_point_ops_emd.emd_forward(p1.to(dev), p2.to(dev))
    assert torch.allclose(loss, (cost / 200).mean())
    gc = torch.full((3,), 1.0 / (200 * 3), device=dev)
    g1, g2 = torch.ops.torch_point_ops_emd.emd_backward(gc, p1.to(dev), p2.to(dev), match)
    assert torch.allclose(a.grad, g1, rtol=1e-6, atol=1e-9)
    assert torch.allclose(b.grad, g2, rtol=1e-6, atol=1e-9)


def test_errors(dev):
    p = torch.randn(1, 8, 3, device=dev)
    with pytest.raises(RuntimeError, match="must be contiguous"):
        torch.ops.torch_point_ops_emd.emd_forward(torch.randn(1, 16, 3, device=dev)[:, ::2], p)
    with pytest.raises(RuntimeError, match="3 channels"):
        torch.ops.torch_point_ops_emd.emd_forward(torch.randn(1, 8, 2, device=dev), p)
    with pytest.raises(RuntimeError, match="same batch size"):
        torch.ops.torch_point_ops_emd.emd_forward(torch.randn(2, 8, 3, device=dev), p)
    with pytest.raises(RuntimeError, match="not implemented for"):
        torch.ops.torch_point_ops_emd.emd_forward(p.bfloat16(), p.bfloat16())


def test_nan_propagates_and_stays_in_its_cloud(O, dev):
    """A NaN coordinate makes its cloud's cost NaN, as in the reference (its
    exponentials turn NaN), while the other clouds are unaffected: the
    kernels' exact skipping of zero exponentials never skips a NaN."""
    p1, p2 = clouds(2, 40, 30, torch.float32, seed=21)
    p1[0, 7, 1] = float("nan")
    cost, match = torch.ops.torch_point_ops_emd.emd_forward(p1.to(dev), p2.to(dev))
    ec, em = O.emd_fwd(np_(p1), np_(p2))
    assert np.isnan(ec[0]) and torch.isnan(cost[0])
    close(np_(match[1]), em[1], *TOL[torch.float32])
    close(np_(cost[1:]), ec[1:], TOL[torch.float32][0], 0.0, scale=1.0)


def test_more_clouds_than_one_launch_holds(O, dev):
    """B = 65537 > 65535 clouds per launch: the entry points run the clouds
    in chunks and reuse the workspace."""
    p1, p2 = clouds(65537, 3, 2, torch.float32, seed=22)
    cost, match = torch.ops.torch_point_ops_emd.emd_forward(p1.to(dev), p2.to(dev))
    ec, em = O.emd_fwd(np_(p1), np_(p2))
    close(np_(match), em, *TOL[torch.float32])
    close(np_(cost), ec, TOL[torch.float32][0], 1e-6, scale=np.abs(ec).max())
    gc = torch.rand(65537, generator=torch.Generator().manual_seed(3))
    g1, g2 = torch.ops.torch_point_ops_emd.emd_backward(gc.to(dev), p1.to(dev), p2.to(dev), match)
    e1, e2 = O.emd_bwd(np_(gc), np_(p1), np_(p2), np_(match))
    close(np_(g1), e1, 1e-4, 1e-4, scale=np.abs(e1).max())
    close(np_(g2), e2, 1e-4, 1e-4, scale=np.abs(e2).max())
