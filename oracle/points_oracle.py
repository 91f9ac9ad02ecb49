"""TEST INFRASTRUCTURE ONLY -- float64 CPU restatement of the reference's
point-sampling front end (Mask2Former-style matching costs on sampled points).

Only ``tests/`` may import this module, and only as the checker; the product
path (``mask_loss_amd``) never imports it.

Coordinates follow the reference's float32 arithmetic (its points are float32
``torch.rand`` draws, and grid_sample unnormalises them in float32), so the
corner cells and the labels under the points are those the reference picks;
the interpolation and the costs are float64.

Pinning (tests/test_oracle_points.py): ``grid_sample_bilinear`` against
``torch.nn.functional.grid_sample`` on the CPU (float64 inputs and
coordinates with ``index_dtype=float64``, float32 ones otherwise), including
zero padding outside the plane; ``point_sample_backward`` against torch's
autograd gradient of the same grid_sample call; ``point_cells`` against the reference's own
torch expression ``clamp(long(x * (W_t - 1)))`` evaluated by torch;
``pairwise_sigmoid_ce_sampling`` / ``pairwise_dice_sampling`` against the
closed forms at z == 0 (BCE = ln 2 * scale for every present class, dice =
(1 - (T + smooth) / (P/2 + T + smooth)) * scale with T points of the class),
the +inf pattern of classes absent from the full label map, and the already
pinned dense pairwise oracle (``mask_oracle.pairwise_sigmoid_ce`` /
``pairwise_dice`` without uncertainty weights) applied to the sampled logits
as a 1 x P map, for the classes present at the points.
"""
from __future__ import annotations

import math

import numpy as np


def _unnormalize(g, size, align_corners, dt):
    """grid_sample's source index of grid coordinate g (reference
    functions/utils.py:17 calls F.grid_sample; PyTorch's
    grid_sampler_unnormalize), in the dtype `dt`."""
    g = g.astype(dt)
    one, half = dt(1.0), dt(0.5)
    if align_corners:
        return ((g + one) * half) * dt(size - 1)
    return ((g + one) * dt(size) - one) * half


def grid_sample_bilinear(inp, grid, align_corners=False, index_dtype=np.float32):
    """torch.nn.functional.grid_sample(inp, grid, mode='bilinear',
    padding_mode='zeros', align_corners) restated: inp (N, C, H, W),
    grid (N, Hg, Wg, 2) of (x, y) in [-1, 1] -> (N, C, Hg, Wg) float64.
    Source indices and corner weights in `index_dtype`, sums in float64."""
    inp = np.asarray(inp, dtype=np.float64)
    N, C, H, W = inp.shape
    dt = index_dtype
    gx = np.asarray(grid[..., 0])
    gy = np.asarray(grid[..., 1])
    ix = _unnormalize(gx, W, align_corners, dt)
    iy = _unnormalize(gy, H, align_corners, dt)
    with np.errstate(invalid="ignore"):
        x0 = np.floor(ix)
        y0 = np.floor(iy)
    x1 = x0 + dt(1.0)
    y1 = y0 + dt(1.0)
    w_nw = ((x1 - ix) * (y1 - iy)).astype(np.float64)
    w_ne = ((ix - x0) * (y1 - iy)).astype(np.float64)
    w_sw = ((x1 - ix) * (iy - y0)).astype(np.float64)
    w_se = ((ix - x0) * (iy - y0)).astype(np.float64)
    out = np.zeros((N, C) + gx.shape[1:], dtype=np.float64)
    for cx, cy, wgt in ((x0, y0, w_nw), (x1, y0, w_ne), (x0, y1, w_sw), (x1, y1, w_se)):
        with np.errstate(invalid="ignore"):
            ok = np.isfinite(cx) & np.isfinite(cy) & (cx >= 0) & (cx <= W - 1) & (cy >= 0) & (cy <= H - 1)
        xi = np.where(ok, cx, 0).astype(np.int64)
        yi = np.where(ok, cy, 0).astype(np.int64)
        for n in range(N):
            v = inp[n][:, yi[n], xi[n]]  # (C, Hg, Wg)
            out[n] += np.where(ok[n][None], v * wgt[n][None], 0.0)
    return out


def point_sample(inp, coords, align_corners=False, index_dtype=np.float32):
    """Reference functions/utils.py:12-20: grid_sample at grid = 2 * coords - 1;
    coords (N, P, 2) -> (N, C, P), or (N, Hg, Wg, 2) -> (N, C, Hg, Wg)."""
    c = np.asarray(coords).astype(index_dtype)
    grid = index_dtype(2.0) * c - index_dtype(1.0)
    if grid.ndim == 3:
        return grid_sample_bilinear(inp, grid[:, :, None, :], align_corners, index_dtype)[..., 0]
    return grid_sample_bilinear(inp, grid, align_corners, index_dtype)


def point_sample_backward(grad_out, coords, H, W, align_corners=False, index_dtype=np.float32):
    """Gradient of point_sample with respect to its (N, C, H, W) input
    (grid_sample's input gradient): every sample's gradient added to its four
    corner cells with the bilinear weights; grad_out (N, C, P) with coords
    (N, P, 2), or (N, C, Hg, Wg) with coords (N, Hg, Wg, 2).  float64 sums."""
    g = np.asarray(grad_out, dtype=np.float64)
    N, C = g.shape[:2]
    g = g.reshape(N, C, -1)
    dt = index_dtype
    c = np.asarray(coords).astype(dt).reshape(N, -1, 2)
    grid = dt(2.0) * c - dt(1.0)
    ix = _unnormalize(grid[..., 0], W, align_corners, dt)
    iy = _unnormalize(grid[..., 1], H, align_corners, dt)
    with np.errstate(invalid="ignore"):
        x0 = np.floor(ix)
        y0 = np.floor(iy)
    x1 = x0 + dt(1.0)
    y1 = y0 + dt(1.0)
    corners = ((x0, y0, (x1 - ix) * (y1 - iy)), (x1, y0, (ix - x0) * (y1 - iy)),
               (x0, y1, (x1 - ix) * (iy - y0)), (x1, y1, (ix - x0) * (iy - y0)))
    out = np.zeros((N, C, H * W), dtype=np.float64)
    for cx, cy, wgt in corners:
        with np.errstate(invalid="ignore"):
            ok = np.isfinite(cx) & np.isfinite(cy) & (cx >= 0) & (cx <= W - 1) & (cy >= 0) & (cy <= H - 1)
        idx = (np.where(ok, cy, 0).astype(np.int64) * W + np.where(ok, cx, 0).astype(np.int64))
        w64 = np.where(ok, wgt.astype(np.float64), 0.0)
        for n in range(N):
            for ch in range(C):
                np.add.at(out[n, ch], idx[n], w64[n] * g[n, ch])
    return out.reshape(N, C, H, W)


def point_cells(x, size):
    """Reference functions/sigmoid/pw_sigmoid_ce.py:499-500:
    clamp(long(x * (size - 1)), 0, size - 1) with x float32; NaN -> 0."""
    f = np.asarray(x, dtype=np.float32) * np.float32(size - 1)
    with np.errstate(invalid="ignore"):
        f = np.where(np.isnan(f), np.float32(0), f)
        t = np.trunc(np.clip(f, -1.0, float(size)))  # clip first: no float -> int overflow
    return np.clip(t.astype(np.int64), 0, size - 1)


def point_labels(targets, coords):
    """Labels under the points, reference functions/sigmoid/pw_sigmoid_ce.py:497-502:
    targets (B, Ht, Wt), coords (B, P, 2) -> (B, P)."""
    targets = np.asarray(targets)
    B, Ht, Wt = targets.shape
    c = np.asarray(coords, dtype=np.float32)
    ix = point_cells(c[..., 0], Wt)
    iy = point_cells(c[..., 1], Ht)
    return np.stack([targets[b][iy[b], ix[b]] for b in range(B)])


def _classes(targets, background_index):
    gt_all = int(np.max(targets)) + 1 if np.size(targets) else 0
    if background_index is None or background_index < 0:
        return gt_all, list(range(max(gt_all, 0)))
    return gt_all, [k for k in range(max(gt_all, 0)) if k != background_index]


def _softplus(x):
    return np.logaddexp(0.0, x)


def pairwise_sigmoid_ce_sampling(logits, targets, coords, background_index=None, scale=1.0,
                                 align_corners=False, gamma=0.0, alpha=None):
    """Reference functions/sigmoid/pw_sigmoid_ce.py:407-550 with the points
    given: logits (L, B, C, h, w), targets (B, Ht, Wt), coords (B, P, 2) ->
    (L, B, C, G) float64, +inf for classes absent from an image's label map
    (:476-484), mean over the points of the focal BCE (:504-536)."""
    logits = np.asarray(logits, dtype=np.float64)
    targets = np.asarray(targets)
    L, B, C, h, w = logits.shape
    gt_all, classes = _classes(targets, background_index)
    col = {k: i for i, k in enumerate(classes)}
    out = np.full((L, B, C, len(classes)), np.inf)
    ap, an = (1.0, 1.0) if alpha is None else (float(alpha), 1.0 - float(alpha))
    labs = point_labels(targets, coords)
    for b in range(B):
        present = [k for k in np.unique(targets[b]).tolist() if k in col]
        if not present:
            continue
        P = coords.shape[1]
        z = point_sample(logits[:, b].reshape(L * C, 1, h, w),
                         np.repeat(np.asarray(coords[b:b + 1]), L * C, axis=0),
                         align_corners)[:, 0, :]  # (L*C, P)
        cp, cn = _softplus(-z), _softplus(z)
        p = 1.0 / (1.0 + np.exp(-z))
        mp, mn = ((1.0 - p) ** gamma, p ** gamma) if gamma != 0.0 else (1.0, 1.0)
        wpos, wneg = ap * mp * cp, an * mn * cn
        for k in present:
            t = (labs[b] == k).astype(np.float64)
            v = (wpos @ t + wneg @ (1.0 - t)) / float(P)
            out[:, b, :, col[k]] = v.reshape(L, C)
    return out * scale


def pairwise_dice_sampling(logits, targets, coords, smooth=1.0, background_index=None, scale=1.0,
                           align_corners=False):
    """Reference functions/dice/pw_dice_loss.py:174-268 with the points given:
    1 - (2 I + smooth) / (P + T + smooth) over the points, +inf for classes
    absent from an image's label map."""
    logits = np.asarray(logits, dtype=np.float64)
    targets = np.asarray(targets)
    L, B, C, h, w = logits.shape
    gt_all, classes = _classes(targets, background_index)
    col = {k: i for i, k in enumerate(classes)}
    out = np.full((L, B, C, len(classes)), np.inf)
    labs = point_labels(targets, coords)
    for b in range(B):
        present = [k for k in np.unique(targets[b]).tolist() if k in col]
        if not present:
            continue
        z = point_sample(logits[:, b].reshape(L * C, 1, h, w),
                         np.repeat(np.asarray(coords[b:b + 1]), L * C, axis=0),
                         align_corners)[:, 0, :]
        p = 1.0 / (1.0 + np.exp(-z))
        psum = p.sum(axis=1)
        for k in present:
            t = (labs[b] == k).astype(np.float64)
            inter = p @ t
            d = 1.0 - (2.0 * inter + smooth) / (psum + t.sum() + smooth)
            out[:, b, :, col[k]] = d.reshape(L, C)
    return out * scale


LN2 = math.log(2.0)
