"""Full-size parity at the BASELINE configurations: every query row, every
cloud, both directions, against the (OpenMP-parallel) oracle.

  config 2  Chamfer B=32, N=M=8192 (fp32 and fp16): forward distances and
            first-index argmin bit for bit, through the op and through the
            fused module loss; the module backward within 1e-5 (fp32) / 1e-2
            (fp16) of the max-abs gradient, against a float64-accumulated
            scatter of the oracle's indices (chamfer.cu:200-234);
  config 3  knn_points B=8, P=16384, K=16, ragged: the raw op output (MinK
            slot layout) bit for bit, the sorted rows equal the reference
            module's torch sort of the oracle's raw output, and return_nn
            equals the reference's gather of those rows;
  config 4  FPS B=16, 65536 -> 4096: all 16 clouds' 4096 samples identical,
            for the uniform+blob cloud and the origin-blob variant (whose
            blob exercises the |p|^2 <= 1e-3 skip rule).
The grid search and bucket pruning kernels are checked here on the exact
inputs the bench times."""
import numpy as np
import pytest
import torch

import workloads

pytestmark = pytest.mark.gpu


def np_(t):
    return t.detach().cpu().numpy()


def assert_bits(got, ref, what):
    got, ref = np.asarray(got), np.asarray(ref)
    assert got.shape == ref.shape and got.dtype == ref.dtype, what
    diff = got.view(np.uint8).reshape(got.shape + (-1,)) != ref.view(np.uint8).reshape(ref.shape + (-1,))
    bad = int(diff.any(-1).sum()) if diff.ndim > got.ndim else int(diff.sum())
    assert bad == 0, f"{what}: {bad} of {got.size} differ"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_config2_forward_every_row_bit_exact(tpo, O, dev, dtype):
    p1, p2 = workloads.chamfer_c2(dtype=dtype)
    print(f"config 2 forward {dtype}: B=32 N=M=8192", flush=True)
    a, b = p1.to(dev), p2.to(dev)
    d1, d2, i1, i2 = torch.ops.torch_point_ops_chamfer.chamfer_forward(a, b)
    loss, k1, k2 = torch.ops.torch_point_ops_chamfer.chamfer_loss_forward(a, b, True)
    e1, e2, j1, j2 = O.chamfer_fwd(np_(p1), np_(p2))
    assert_bits(np_(d1), e1, "dist1")
    assert_bits(np_(d2), e2, "dist2")
    assert_bits(np_(i1), j1, "idx1")
    assert_bits(np_(i2), j2, "idx2")
    assert_bits(np_(k1), j1, "module idx1")
    assert_bits(np_(k2), j2, "module idx2")
    want = e1.astype(np.float64).mean() + e2.astype(np.float64).mean()
    tol = 1e-3 if dtype == torch.float16 else 1e-5
    assert abs(float(loss) - want) <= tol * want


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_config2_module_backward(tpo, O, dev, dtype):
    p1, p2 = workloads.chamfer_c2(dtype=dtype)
    print(f"config 2 backward {dtype}: B=32 N=M=8192", flush=True)
    a = p1.to(dev).requires_grad_(True)
    b = p2.to(dev).requires_grad_(True)
    tpo.ChamferDistance("mean")(a, b).backward()
    _, _, j1, j2 = O.chamfer_fwd(np_(p1), np_(p2))
    npdt = np.float16 if dtype == torch.float16 else np.float32
    # MeanBackward spreads g * (1/numel), rounded to the dtype
    g1 = np.full(j1.shape, npdt(1.0 / j1.size), npdt)
    g2 = np.full(j2.shape, npdt(1.0 / j2.size), npdt)
    ea, eb = O.chamfer_bwd(np_(p1), np_(p2), j1, j2, g1, g2, accum_f64=True)
    tol = 1e-2 if dtype == torch.float16 else 1e-5
    for got, ref in ((np_(a.grad), ea), (np_(b.grad), eb)):
        err = np.abs(got.astype(np.float64) - ref.astype(np.float64)).max()
        assert err <= tol * np.abs(ref.astype(np.float64)).max(), err


def _module_sort(idxs, dists, lengths2, K):
    # the reference's knn_points sort after the forward (knn/__init__.py:111-131)
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


def test_config3_every_row_raw_sorted_and_return_nn(tpo, O, dev):
    p1, p2, l1, l2 = workloads.knn_c3()
    print("config 3: B=8 P=16384 K=16 ragged", flush=True)
    a, b, la, lb = p1.to(dev), p2.to(dev), l1.to(dev), l2.to(dev)
    ri, rd = torch.ops.torch_point_ops_knn.knn_forward(a, b, la, lb, 2, 16, -1)
    ei, ed = O.knn_fwd(np_(p1), np_(p2), np_(l1), np_(l2), norm=2, K=16)
    assert_bits(np_(ri), ei, "raw idxs")
    assert_bits(np_(rd), ed, "raw dists")
    # the module (KNearestNeighbors(K=16, return_nn=True) is knn_points +
    # knn_gather): sorted rows equal the reference's sort of the oracle rows
    want_i, want_d = _module_sort(torch.from_numpy(ei).to(dev), torch.from_numpy(ed).to(dev), lb, 16)
    idx, d, nn = tpo.KNearestNeighbors(K=16, return_nn=True)(a, b, la, lb)
    assert torch.equal(idx, want_i) and torch.equal(d, want_d)
    U = b.shape[2]
    want_nn = b[:, :, None].expand(-1, -1, 16, -1).gather(1, want_i[..., None].expand(-1, -1, -1, U))
    pad = lb[:, None] <= torch.arange(16, device=dev)[None]
    want_nn[pad[:, None].expand(-1, want_i.shape[1], -1)] = 0
    assert torch.equal(nn, want_nn)


@pytest.mark.parametrize("origin_blob", [False, True])
def test_config4_all_clouds_all_samples(tpo, O, dev, origin_blob):
    pts = workloads.fps_c4(origin_blob=origin_blob)
    print(f"config 4: B=16 N=65536 -> 4096 origin_blob={origin_blob}", flush=True)
    idx = tpo.furthest_point_sampling(pts.to(dev), 4096)
    ref = O.fps(np_(pts), 4096)
    got = np_(idx)
    bad = [b for b in range(pts.shape[0]) if not np.array_equal(got[b], ref[b])]
    assert not bad, f"clouds {bad} differ"
    if origin_blob:  # the skip rule is live: some points take no part
        mag = (pts.double() ** 2).sum(-1)
        assert bool((mag <= 1e-3).any())
        assert bool((torch.gather(mag, 1, idx.cpu())[:, 1:] > 1e-3 * (1 - 1e-6)).all())
