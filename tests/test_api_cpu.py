"""Host-side API checks that need no GPU: operator schemas (verbatim from the
reference), Python-level validation (the reference's ValueErrors) and the
CPU behaviour of chamfer (the reference has no CPU kernel)."""
import pytest
import torch


def test_schemas_match_reference(tpo):
    ops = torch.ops
    # chamfer.cpp:35-38, knn.cpp:168-171, fps.cpp:159-161, fps.cpp:166
    want = {
        ops.torch_point_ops_chamfer.chamfer_forward:
            "chamfer_forward(Tensor xyz1, Tensor xyz2) -> (Tensor, Tensor, Tensor, Tensor)",
        ops.torch_point_ops_chamfer.chamfer_backward:
            "chamfer_backward(Tensor xyz1, Tensor xyz2, Tensor idx1, Tensor idx2, "
            "Tensor grad_dist1, Tensor grad_dist2) -> (Tensor, Tensor)",
        ops.torch_point_ops_knn.knn_forward:
            "knn_forward(Tensor p1, Tensor p2, Tensor lengths1, Tensor lengths2, int norm, "
            "int K, int version) -> (Tensor, Tensor)",
        ops.torch_point_ops_knn.knn_backward:
            "knn_backward(Tensor p1, Tensor p2, Tensor lengths1, Tensor lengths2, Tensor idxs, "
            "int norm, Tensor grad_dists) -> (Tensor, Tensor)",
        ops.torch_point_ops_fps.fps_forward: "fps_forward(Tensor points, int nsamples) -> Tensor",
        ops.torch_point_ops_fps.gather_points_forward:
            "gather_points_forward(Tensor points, Tensor idx) -> Tensor",
        ops.torch_point_ops_fps.gather_points_backward:
            "gather_points_backward(Tensor grad_out, Tensor idx, int n) -> Tensor",
        ops.torch_point_ops_quick_fps.quick_fps_forward:
            "quick_fps_forward(Tensor points, int nsamples, int kd_depth=4) -> Tensor",
        # emd.cpp:32-33
        ops.torch_point_ops_emd.emd_forward:
            "emd_forward(Tensor xyz1, Tensor xyz2) -> (Tensor, Tensor)",
        ops.torch_point_ops_emd.emd_backward:
            "emd_backward(Tensor grad_cost, Tensor xyz1, Tensor xyz2, Tensor match) -> "
            "(Tensor, Tensor)",
    }
    for op, schema in want.items():
        s = str(op.default._schema)
        assert s.split("::", 1)[-1] == schema


def test_fused_ops_schemas_and_fake_kernels(tpo):
    # the extra ops behind ChamferDistance's reduction and knn_points' sort
    # and gather: schemas, and FakeTensor shapes (what torch.compile traces)
    from torch._subclasses.fake_tensor import FakeTensorMode

    ops = torch.ops
    want = {
        ops.torch_point_ops_chamfer.chamfer_loss_forward:
            "chamfer_loss_forward(Tensor xyz1, Tensor xyz2, bool mean) -> (Tensor, Tensor, Tensor)",
        ops.torch_point_ops_chamfer.chamfer_loss_backward:
            "chamfer_loss_backward(Tensor xyz1, Tensor xyz2, Tensor idx1, Tensor idx2, "
            "Tensor grad_loss, bool mean) -> (Tensor, Tensor)",
        ops.torch_point_ops_knn.knn_forward_sorted:
            "knn_forward_sorted(Tensor p1, Tensor p2, Tensor lengths1, Tensor lengths2, "
            "int norm, int K, int version) -> (Tensor, Tensor)",
        ops.torch_point_ops_knn.knn_gather:
            "knn_gather(Tensor x, Tensor idx, Tensor lengths) -> Tensor",
    }
    for op, schema in want.items():
        assert str(op.default._schema).split("::", 1)[-1] == schema
    with FakeTensorMode():
        a, b = torch.empty(2, 7, 3), torch.empty(2, 5, 3)
        loss, i1, i2 = ops.torch_point_ops_chamfer.chamfer_loss_forward(a, b, True)
        assert loss.shape == () and i1.shape == (2, 7) and i2.shape == (2, 5)
        assert i1.dtype == torch.int32
        l1 = torch.empty(2, dtype=torch.int64)
        idx, d = ops.torch_point_ops_knn.knn_forward_sorted(a, b, l1, l1, 2, 4, -1)
        assert idx.shape == (2, 7, 4) and idx.dtype == torch.int64 and d.dtype == a.dtype
        nn = ops.torch_point_ops_knn.knn_gather(b, idx, l1)
        assert nn.shape == (2, 7, 4, 3)


def test_chamfer_loss_cpu_not_implemented(tpo):
    a = torch.zeros(1, 2, 3, requires_grad=True)
    for red in ("mean", "sum"):
        with pytest.raises(RuntimeError, match="not implemented for CPU"):
            tpo.ChamferDistance(red)(a, torch.zeros(1, 2, 3))


def test_public_names(tpo):
    for name in ("ChamferDistance", "chamfer_distance", "KNearestNeighbors", "knn_points",
                 "knn_gather", "FarthestPointSampling", "furthest_point_sampling",
                 "gather_points", "farthest_point_sample_and_gather",
                 "QuickFarthestPointSampling", "quick_furthest_point_sampling",
                 "quick_farthest_point_sample_and_gather", "EarthMoverDistance", "emd",
                 "chamfer_loss",
                 "earth_movers_distance"):
        assert hasattr(tpo, name)
    from torch_point_ops.fps import FPSFunction, PointGatherer, fps_function  # noqa: F401
    from torch_point_ops.knn import KNNFunction  # noqa: F401


def test_chamfer_cpu_not_implemented(tpo):
    with pytest.raises(RuntimeError, match="not implemented for CPU"):
        tpo.chamfer_distance(torch.zeros(1, 2, 3), torch.zeros(1, 2, 3))


def test_emd_cpu_not_implemented(tpo):
    # emd.cpp:19-28
    with pytest.raises(RuntimeError, match="emd_forward is not implemented for CPU"):
        tpo.earth_movers_distance(torch.zeros(1, 2, 3), torch.zeros(1, 2, 3))
    with pytest.raises(RuntimeError, match="emd_backward is not implemented for CPU"):
        torch.ops.torch_point_ops_emd.emd_backward(torch.zeros(1), torch.zeros(1, 2, 3),
                                                   torch.zeros(1, 2, 3), torch.zeros(1, 2, 2))
    assert tpo.emd is tpo.earth_movers_distance
    from torch_point_ops.emd.emd import EarthMoverDistance

    assert EarthMoverDistance is tpo.EarthMoverDistance


def test_validation_errors(tpo):
    p = torch.zeros(1, 10, 3)
    with pytest.raises(ValueError):
        tpo.furthest_point_sampling(p.squeeze(0), 5)
    with pytest.raises(ValueError):
        tpo.furthest_point_sampling(p[..., :2], 5)
    with pytest.raises(ValueError):
        tpo.furthest_point_sampling(p, 0)
    with pytest.raises(ValueError):
        tpo.furthest_point_sampling(p, 15)
    with pytest.raises(ValueError):
        tpo.quick_furthest_point_sampling(p, 5, kd_depth=11)
    f = torch.zeros(2, 6, 20)
    i = torch.zeros(2, 8, dtype=torch.long)
    with pytest.raises(ValueError):
        tpo.gather_points(f[0], i)
    with pytest.raises(ValueError):
        tpo.gather_points(f, i.unsqueeze(-1))
    with pytest.raises(ValueError):
        tpo.gather_points(f, i[:1])
    with pytest.raises(ValueError):
        tpo.knn_points(torch.zeros(2, 4, 3), torch.zeros(1, 4, 3))
    with pytest.raises(ValueError):
        tpo.knn_points(torch.zeros(1, 4, 3), torch.zeros(1, 4, 2))
    with pytest.raises(ValueError):
        tpo.KNearestNeighbors(K=0)
    with pytest.raises(ValueError):
        tpo.KNearestNeighbors(norm=3)
    with pytest.raises(ValueError):
        tpo.ChamferDistance(reduction="max")
    with pytest.raises(ValueError):
        tpo.FarthestPointSampling(0)


def test_fake_kernels(tpo):
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        a = torch.empty(2, 5, 3)
        b = torch.empty(2, 7, 3)
        d1, d2, i1, i2 = torch.ops.torch_point_ops_chamfer.chamfer_forward(a, b)
        assert d1.shape == (2, 5) and i2.shape == (2, 7) and i1.dtype == torch.int32
        idx, d = torch.ops.torch_point_ops_knn.knn_forward(
            a, b, torch.empty(2, dtype=torch.long), torch.empty(2, dtype=torch.long), 2, 4, -1)
        assert idx.shape == (2, 5, 4) and idx.dtype == torch.int64 and d.dtype == a.dtype
        s = torch.ops.torch_point_ops_fps.fps_forward(b, 3)
        assert s.shape == (2, 3) and s.dtype == torch.int64
        g = torch.ops.torch_point_ops_fps.gather_points_forward(torch.empty(2, 6, 7), s)
        assert g.shape == (2, 6, 3)
        gb = torch.ops.torch_point_ops_fps.gather_points_backward(g, s, 7)
        assert gb.shape == (2, 6, 7)
        cost, match = torch.ops.torch_point_ops_emd.emd_forward(a, b)
        assert cost.shape == (2,) and match.shape == (2, 7, 5) and match.dtype == a.dtype
        g1, g2 = torch.ops.torch_point_ops_emd.emd_backward(cost, a, b, match)
        assert g1.shape == a.shape and g2.shape == b.shape
