"""A second, independent statement of the reference's approximate EMD
(emd.cu:18-230 approxmatch + matchcost, :234-303 matchcostgrad1/2),
vectorised over both clouds with numpy, used only to pin the C oracle.

It is written from the reference's algorithm, not from the oracle: a
mistake in the level schedule, the regularisers, the order of the three
passes per level or the narrowing of double arguments by the reference's
fminf/fmaxf would have to be made twice, differently, to pass both.  The
sums run in numpy's order, so results agree with the oracle to rounding
(float64) or to float32 accumulation differences (float32)."""
import numpy as np


def _sqdist(x1, x2):
    # (x2 - x1)^2 + (y2 - y1)^2 + (z2 - z1)^2, left to right (emd.cu:70);
    # (n, m) for x1 (n, 3), x2 (m, 3)
    dx = x2[None, :, 0] - x1[:, None, 0]
    dy = x2[None, :, 1] - x1[:, None, 1]
    dz = x2[None, :, 2] - x1[:, None, 2]
    return dx * dx + dy * dy + dz * dz


def emd_forward(xyz1, xyz2, levels=range(7, -3, -1)):
    """-> (cost[B], match[B, m, n]) in the inputs' dtype (float32 or float64:
    opmath is the type itself).  `levels` is the reference's exponent
    schedule (j = 7 .. -2, the last one meaning level 0); tests pass another
    one to show that a slip in it is detected."""
    t = xyz1.dtype.type
    f32 = np.float32
    B, n, _ = xyz1.shape
    m = xyz2.shape[1]
    # emd.cu:22-28: float(n) / m is a float division, stored as scalar_t
    if n >= m:
        multi_l, multi_r = t(1), t(f32(n) / f32(m))
    else:
        multi_l, multi_r = t(f32(m) / f32(n)), t(1)
    eps = t(f32(1e-9))  # static_cast<opmath_t>(1e-9f)
    cost = np.zeros(B, xyz1.dtype)
    match = np.zeros((B, m, n), xyz1.dtype)
    for b in range(B):
        x1, x2 = xyz1[b], xyz2[b]
        d = _sqdist(x1, x2)  # (n, m)
        remain_l = np.full(n, multi_l, xyz1.dtype)
        remain_r = np.full(m, multi_r, xyz1.dtype)
        for j in levels:  # -4^7 .. -4^-1, then 0
            level = t(0) if j == -2 else -t(4.0) ** t(j)
            w = np.exp(level * d)  # (n, m)
            # pass 1: each xyz1 point's share of its remaining mass
            suml = eps + (w * remain_r[None, :]).sum(1, dtype=xyz1.dtype)
            ratio_l = remain_l / (suml + eps)
            # pass 2: each xyz2 point's consumption; fminf / fmaxf take float
            sumr = (w * ratio_l[:, None]).sum(0, dtype=xyz1.dtype) * remain_r
            consumption = np.minimum((remain_r / (sumr + eps)).astype(f32), f32(1)).astype(xyz1.dtype)
            ratio_r = consumption * remain_r
            remain_r = np.maximum(f32(0), (remain_r - sumr).astype(f32)).astype(xyz1.dtype)
            # pass 3: the flow of this level, and what it takes from xyz1's points
            flow = w * ratio_l[:, None] * ratio_r[None, :]  # (n, m)
            match[b] += flow.T
            remain_l = np.maximum(f32(0), (remain_l - flow.sum(1, dtype=xyz1.dtype)).astype(f32)
                                  ).astype(xyz1.dtype)
        cost[b] = (d * match[b].T).sum(dtype=xyz1.dtype)
    return cost, match


def emd_backward(grad_cost, xyz1, xyz2, match):
    """-> (grad_xyz1, grad_xyz2): 2 * match-weighted coordinate differences
    times the upstream gradient of each cloud's cost."""
    g1 = np.empty_like(xyz1)
    g2 = np.empty_like(xyz2)
    for b in range(xyz1.shape[0]):
        x1, x2, mt = xyz1[b], xyz2[b], match[b]  # mt: (m, n)
        two = mt.T * 2  # (n, m)
        diff = x1[:, None, :] - x2[None, :, :]  # (n, m, 3)
        g1[b] = (diff * two[..., None]).sum(1) * grad_cost[b]
        g2[b] = (-diff * two[..., None]).sum(0) * grad_cost[b]
    return g1, g2
