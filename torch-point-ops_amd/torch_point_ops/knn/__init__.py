"""K nearest neighbours (reference: torch_point_ops/knn/__init__.py:1-187).

torch.ops.torch_point_ops_knn.knn_forward / knn_backward run the gfx950
kernels of libtpo_hip.so; knn_points adds the reference's validation,
default lengths and sorting, knn_gather the gather of neighbour features.
"""
import torch

from .. import _C  # noqa: F401


def _knn_backward(ctx, grad_idxs, grad_dists):
    p1, p2, lengths1, lengths2, idxs = ctx.saved_tensors
    if grad_dists is None:  # gradients are not materialised: the index output has none
        return None, None, None, None, None, None, None
    grad_p1, grad_p2 = torch.ops.torch_point_ops_knn.knn_backward(
        p1, p2, lengths1, lengths2, idxs, ctx.norm, grad_dists
    )
    # no gradient for lengths1, lengths2, norm, K, version
    return grad_p1, grad_p2, None, None, None, None, None


def _knn_setup_context(ctx, inputs, output):
    p1, p2, lengths1, lengths2, norm, _K, _version = inputs
    idxs, _dists = output
    ctx.save_for_backward(p1, p2, lengths1, lengths2, idxs)
    ctx.norm = norm
    ctx.set_materialize_grads(False)  # no zero tensor for the index output


torch.library.register_autograd(
    "torch_point_ops_knn::knn_forward", _knn_backward, setup_context=_knn_setup_context
)
# the sorted forward's rows are a permutation of knn_forward's: same gradient
torch.library.register_autograd(
    "torch_point_ops_knn::knn_forward_sorted", _knn_backward, setup_context=_knn_setup_context
)


@torch.library.register_fake("torch_point_ops_knn::knn_forward")
def _knn_forward_fake(p1, p2, lengths1, lengths2, norm, K, version):
    n, p = p1.shape[0], p1.shape[1]
    return (
        torch.empty(n, p, K, device=p1.device, dtype=torch.int64),
        torch.empty(n, p, K, device=p1.device, dtype=p1.dtype),
    )


@torch.library.register_fake("torch_point_ops_knn::knn_forward_sorted")
def _knn_forward_sorted_fake(p1, p2, lengths1, lengths2, norm, K, version):
    return _knn_forward_fake(p1, p2, lengths1, lengths2, norm, K, version)


# dtypes whose sorted rows come straight from the kernel (2 <= K <= 32)
_SORTED_IN_KERNEL = (torch.float32, torch.float64, torch.float16)


def _knn_gather_backward(ctx, grad_out):
    # gather's gradient: scatter-add the rows back (the masked slots carry none)
    idx, lengths = ctx.saved_tensors
    if grad_out is None or not ctx.needs_input_grad[0]:
        return None, None, None
    N, L, K, U = grad_out.shape
    keep = (torch.arange(K, device=idx.device)[None] < lengths[:, None])[:, None, :, None]
    g = (grad_out * keep).reshape(N, L * K, U)
    j = idx.clamp(0, ctx.M - 1).reshape(N, L * K, 1).expand(-1, -1, U)
    grad_x = torch.zeros(N, ctx.M, U, dtype=grad_out.dtype, device=grad_out.device)
    return grad_x.scatter_add_(1, j, g), None, None


def _knn_gather_setup_context(ctx, inputs, output):
    x, idx, lengths = inputs
    ctx.save_for_backward(idx, lengths)
    ctx.M = x.shape[1]


torch.library.register_autograd(
    "torch_point_ops_knn::knn_gather", _knn_gather_backward,
    setup_context=_knn_gather_setup_context,
)


@torch.library.register_fake("torch_point_ops_knn::knn_gather")
def _knn_gather_fake(x, idx, lengths):
    return x.new_empty(idx.shape[0], idx.shape[1], idx.shape[2], x.shape[2])


@torch.library.register_fake("torch_point_ops_knn::knn_backward")
def _knn_backward_fake(p1, p2, lengths1, lengths2, idxs, norm, grad_dists):
    return torch.empty_like(p1), torch.empty_like(p2)


def knn_points(
    p1: torch.Tensor,
    p2: torch.Tensor,
    lengths1: torch.Tensor = None,
    lengths2: torch.Tensor = None,
    norm: int = 2,
    K: int = 1,
    version: int = -1,
    return_sorted: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    """K nearest neighbours of every point of p1 among the points of p2.

    Args:
        p1: (N, P1, D) query clouds; p2: (N, P2, D) reference clouds.
        lengths1, lengths2: (N,) int64 valid point counts (default: all points).
        norm: 2 for squared L2 distances, 1 for L1.
        K: neighbours per query.
        version: kernel semantics to reproduce (-1 automatic, 0..3).
        return_sorted: sort each row by distance (slots past lengths2 last).

    Returns:
        idxs (N, P1, K) int64 and dists (N, P1, K) in the input dtype.
    """
    if p1.shape[0] != p2.shape[0]:
        raise ValueError("p1 and p2 must have the same batch dimension.")
    if p1.shape[2] != p2.shape[2]:
        raise ValueError("p1 and p2 must have the same point dimension.")
    N, P1, _D = p1.shape
    P2 = p2.shape[1]
    if lengths1 is None:
        lengths1 = torch.full((N,), P1, dtype=torch.int64, device=p1.device)
    if lengths2 is None:
        lengths2 = torch.full((N,), P2, dtype=torch.int64, device=p1.device)

    if return_sorted and 2 <= K <= 32 and p1.dtype in _SORTED_IN_KERNEL and p1.is_cuda:
        # the kernel replays the sort below (torch's network, ties included)
        return torch.ops.torch_point_ops_knn.knn_forward_sorted(
            p1.contiguous(), p2.contiguous(), lengths1.contiguous(), lengths2.contiguous(),
            norm, K, version,
        )

    idxs, dists = torch.ops.torch_point_ops_knn.knn_forward(
        p1.contiguous(), p2.contiguous(), lengths1.contiguous(), lengths2.contiguous(),
        norm, K, version,
    )

    if K > 1 and return_sorted:
        # slots k >= lengths2[n] hold padding: sort them last, report them as 0
        # (reference knn/__init__.py:111-131)
        if lengths2.min() < K:
            pad = lengths2[:, None] <= torch.arange(K, device=dists.device)[None]
            pad = pad[:, None].expand(-1, P1, -1)
            keyed = dists.clone()
            keyed[pad] = torch.tensor(float("inf"), dtype=dists.dtype, device=dists.device)
            dists, order = keyed.sort(dim=2)
            dists[pad] = torch.tensor(0, dtype=dists.dtype, device=dists.device)
        else:
            dists, order = dists.sort(dim=2)
        idxs = idxs.gather(2, order)
    return idxs, dists


def knn_gather(x: torch.Tensor, idx: torch.Tensor, lengths: torch.Tensor = None) -> torch.Tensor:
    """x_out[n, l, k] = x[n, idx[n, l, k]], zero for k >= lengths[n].

    Args:
        x: (N, M, U) features; idx: (N, L, K) indices from knn_points;
        lengths: (N,) valid counts of x (default M).

    Returns:
        (N, L, K, U) gathered features (reference knn/__init__.py:136-183).
    """
    N, M, U = x.shape
    _N, L, K = idx.shape
    if N != _N:
        raise ValueError("x and idx must have same batch dimension.")
    if lengths is None:
        lengths = torch.full((N,), M, dtype=torch.int64, device=x.device)
    if x.is_cuda and M > 0:
        # one kernel for the gather and the mask below (no host-side test)
        return torch.ops.torch_point_ops_knn.knn_gather(x, idx, lengths.to(torch.int64))
    expanded = idx[:, :, :, None].expand(-1, -1, -1, U)
    out = x[:, :, None].expand(-1, -1, K, -1).gather(1, expanded)
    if lengths.min() < K:
        pad = lengths[:, None] <= torch.arange(K, device=x.device)[None]
        pad = pad[:, None].expand(-1, L, -1)[:, :, :, None].expand(-1, -1, -1, U)
        out[pad] = torch.tensor(0, dtype=x.dtype, device=x.device)
    return out


from .knn import KNearestNeighbors, KNNFunction, knn_function  # noqa: E402
