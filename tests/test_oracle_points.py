"""CPU pinning of the point-sampling oracle (oracle/points_oracle.py).

* grid_sample_bilinear / point_sample: torch.nn.functional.grid_sample on the
  CPU (a library routine, the function the reference's point_sample calls,
  functions/utils.py:17), float64 with float64 indices to 1e-12 and float32
  to float32 rounding, inside and outside the plane, both align_corners.
* point_sample_backward: torch's autograd gradient of the same grid_sample
  call (float64, both align_corners, points outside the plane).
* point_cells / point_labels: the reference's own expression
  clamp(long(x * (W_t - 1)), 0, W_t - 1) evaluated by torch in float32,
  including the borders and coordinates outside [0, 1].
* sampling costs: closed forms at z == 0, the +inf pattern of classes absent
  from the full label map, and the dense pairwise oracle (already pinned in
  tests/test_oracle.py) on the sampled logits as a 1 x P map.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import mask_oracle as MO
from oracle import points_oracle as PO


def _coords(rng, N, P, lo=0.0, hi=1.0):
    return rng.uniform(lo, hi, size=(N, P, 2)).astype(np.float32)


@pytest.mark.parametrize("align", [False, True])
@pytest.mark.parametrize("H,W", [(7, 5), (16, 16), (1, 9)])
def test_grid_sample_matches_torch_float64(align, H, W):
    rng = np.random.default_rng(H * 31 + W + align)
    inp = rng.normal(0, 2, size=(3, 4, H, W))
    # inside, on the border and outside the plane
    c = _coords(rng, 3, 200, -0.3, 1.3).astype(np.float64)
    c[0, :4] = [[0, 0], [1, 1], [0.5, 0.5], [1, 0]]
    got = PO.point_sample(inp, c, align, index_dtype=np.float64)
    ref = F.grid_sample(torch.from_numpy(inp), torch.from_numpy(2.0 * c - 1.0)[:, :, None, :],
                        mode="bilinear", padding_mode="zeros", align_corners=align)[..., 0].numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("align", [False, True])
def test_grid_sample_matches_torch_float32_and_4d_grid(align):
    rng = np.random.default_rng(5 + align)
    inp = rng.normal(0, 3, size=(2, 3, 12, 10)).astype(np.float32)
    c = _coords(rng, 2, 6 * 7, -0.1, 1.1).reshape(2, 6, 7, 2)
    got = PO.point_sample(inp, c, align)
    ref = F.grid_sample(torch.from_numpy(inp), 2.0 * torch.from_numpy(c) - 1.0, mode="bilinear",
                        padding_mode="zeros", align_corners=align).numpy()
    assert got.shape == ref.shape == (2, 3, 6, 7)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("align", [False, True])
def test_point_sample_backward_matches_torch_autograd(align):
    rng = np.random.default_rng(17 + align)
    H, W = 7, 9
    inp = torch.from_numpy(rng.normal(size=(2, 3, H, W))).requires_grad_(True)
    c = _coords(rng, 2, 150, -0.2, 1.2).astype(np.float64)
    c[0, :3] = [[0, 0], [1, 1], [0.5, 0.25]]
    out = F.grid_sample(inp, torch.from_numpy(2.0 * c - 1.0)[:, :, None, :], mode="bilinear",
                        padding_mode="zeros", align_corners=align)[..., 0]
    g = rng.normal(size=out.shape)
    out.backward(torch.from_numpy(g))
    got = PO.point_sample_backward(g, c, H, W, align, index_dtype=np.float64)
    np.testing.assert_allclose(got, inp.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_grid_sample_exact_at_cell_centres():
    # align_corners=False: coordinate (j + 0.5) / W samples cell j exactly
    rng = np.random.default_rng(0)
    H, W = 6, 8
    inp = rng.normal(size=(1, 2, H, W))
    ys, xs = np.meshgrid(np.arange(H), np.arange(W), indexing="ij")
    c = np.stack([(xs + 0.5) / W, (ys + 0.5) / H], -1).reshape(1, -1, 2)
    got = PO.point_sample(inp, c, False, index_dtype=np.float64)
    np.testing.assert_allclose(got.reshape(1, 2, H, W), inp, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("size", [1, 2, 7, 256, 1000])
def test_point_cells_match_reference_expression(size):
    rng = np.random.default_rng(size)
    x = np.concatenate([rng.uniform(-0.5, 1.5, 4000), np.arange(size) / max(size - 1, 1),
                        [0.0, 1.0, -0.0, 1e-8, 1 - 1e-7, np.nextafter(np.float32(1), 0)]]).astype(np.float32)
    ref = torch.clamp((torch.from_numpy(x) * (size - 1)).long(), 0, size - 1).numpy()
    np.testing.assert_array_equal(PO.point_cells(x, size), ref)


def test_point_labels_index_rows_and_columns():
    rng = np.random.default_rng(3)
    t = rng.integers(0, 9, size=(2, 5, 7))
    c = _coords(rng, 2, 300)
    lab = PO.point_labels(t, c)
    tt = torch.from_numpy(t)
    for b in range(2):
        xy = torch.from_numpy(c[b])
        ix = torch.clamp((xy[:, 0] * (7 - 1)).long(), 0, 7 - 1)
        iy = torch.clamp((xy[:, 1] * (5 - 1)).long(), 0, 5 - 1)
        np.testing.assert_array_equal(lab[b], tt[b][iy, ix].numpy())


def _case(seed, L=2, B=3, C=4, h=6, w=5, Ht=12, Wt=10, G=5, P=97):
    rng = np.random.default_rng(seed)
    z = rng.normal(0, 2, size=(L, B, C, h, w))
    t = rng.integers(0, G + 1, size=(B, Ht, Wt))
    t[1] = np.where(t[1] == 3, 0, t[1])  # class 3 absent from image 1
    t[2, 0, 0] = G                        # class G present in image 2 at one pixel
    c = _coords(rng, B, P)
    return z, t, c


@pytest.mark.parametrize("bg", [None, 0])
def test_sampling_costs_closed_forms_at_zero_logits(bg):
    z, t, c = _case(1)
    z[:] = 0.0
    P = c.shape[1]
    bce = PO.pairwise_sigmoid_ce_sampling(z, t, c, background_index=bg, scale=2.0)
    dice = PO.pairwise_dice_sampling(z, t, c, smooth=1.0, background_index=bg, scale=3.0)
    labs = PO.point_labels(t, c)
    classes = [k for k in range(int(t.max()) + 1) if bg is None or k != bg]
    for b in range(t.shape[0]):
        for i, k in enumerate(classes):
            if not (t[b] == k).any():
                assert np.isinf(bce[:, b, :, i]).all() and np.isinf(dice[:, b, :, i]).all()
                continue
            T = float((labs[b] == k).sum())
            np.testing.assert_allclose(bce[:, b, :, i], 2.0 * PO.LN2, rtol=1e-14)
            np.testing.assert_allclose(dice[:, b, :, i], 3.0 * (1.0 - (T + 1.0) / (P / 2 + T + 1.0)),
                                       rtol=1e-14)


def test_sampling_costs_absent_class_and_width():
    z, t, c = _case(2)
    bce = PO.pairwise_sigmoid_ce_sampling(z, t, c, background_index=0)
    assert bce.shape[-1] == int(t.max())  # classes 1..max
    assert np.isinf(bce[:, 1, :, 3 - 1]).all()      # class 3 absent from image 1
    assert np.isfinite(bce[:, 2, :, -1]).all()      # present at one pixel: finite


@pytest.mark.parametrize("gamma,alpha", [(0.0, None), (2.0, 0.25)])
def test_sampling_costs_equal_dense_oracle_on_sampled_map(gamma, alpha):
    z, t, c = _case(4)
    L, B, C = z.shape[:3]
    P = c.shape[1]
    bce = PO.pairwise_sigmoid_ce_sampling(z, t, c, gamma=gamma, alpha=alpha, scale=1.5)
    dice = PO.pairwise_dice_sampling(z, t, c, smooth=0.5, scale=1.5)
    zs = np.stack([PO.point_sample(z[:, b].reshape(L * C, 1, *z.shape[3:]),
                                   np.repeat(c[b:b + 1], L * C, axis=0))[:, 0, :].reshape(L, C, P)
                   for b in range(B)], axis=1)[:, :, :, None, :]  # (L, B, C, 1, P)
    labs = PO.point_labels(t, c)[:, None, :]
    GT = int(t.max()) + 1
    # GT width from the full map (the points may miss the top label)
    dense_b, _ = MO.pairwise_mask_costs(zs, labs, GT, -1, 1.0, 1.5, 1.0, 0.0, 0.0, gamma,
                                        -1.0 if alpha is None else alpha, False)
    _, dense_d = MO.pairwise_mask_costs(zs, labs, GT, -1, 0.5, 1.0, 1.5, 0.0, 0.0)
    for b in range(B):
        for k in range(GT):
            if (labs[b] == k).any():  # present at the points: both definitions apply
                np.testing.assert_allclose(bce[:, b, :, k], dense_b[:, b, :, k], rtol=1e-11)
                np.testing.assert_allclose(dice[:, b, :, k], dense_d[:, b, :, k], rtol=1e-11)
