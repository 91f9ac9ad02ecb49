"""CPU checks that pin the oracle's standalone operators before they serve as
the parity reference of the HIP path:

=====================================  ==============================================
oracle function                        pinned by
=====================================  ==============================================
gt_total_from_targets                  hand examples (max + 1, empty, all negative)
pairwise_sigmoid_ce, pairwise_dice     naive high-resolution evaluation on nearest-
                                       upsampled logits (tests/test_oracle.py's
                                       naive_costs, scipy terms, no counts) with
                                       GT slots 0..max(targets)
sigmoid_ce_loss                        naive high-resolution one-hot evaluation
                                       (scipy log_expit / expit); closed form at
                                       z == 0: B C ln2 scale / num_masks
sigmoid_ce_backward                    central finite differences of the naive loss
dice_loss (loss, I, P, T)              naive high-resolution one-hot sums; closed
                                       form at z == 0
dice_loss_backward                     central finite differences of the naive loss
=====================================  ==============================================
"""
import math

import numpy as np
import pytest
from scipy import special

from oracle import mask_oracle as O

from test_oracle import naive_costs


def upsample(z, s):
    return np.repeat(np.repeat(z, s, axis=-2), s, axis=-1)


def naive_sigmoid_ce(z, tgt, num_masks, scale=1.0, gamma=0.0, alpha=-1.0):
    """Per-pixel focal BCE with explicit upsampling and one-hot targets
    (independent of the count formulation)."""
    L, B, C, H, W = z.shape
    Ht, Wt = tgt.shape[1:]
    zu = upsample(z, Ht // H)
    y = np.stack([(tgt == c) for c in range(C)], axis=1).astype(np.float64)[None]
    p = special.expit(zu)
    cp = -special.log_expit(zu)
    cn = -special.log_expit(-zu)
    mp = (1 - p) ** gamma if gamma > 0 else 1.0
    mn = p ** gamma if gamma > 0 else 1.0
    ap, an = (alpha, 1 - alpha) if alpha >= 0 else (1.0, 1.0)
    loss = ap * y * mp * cp + an * (1 - y) * mn * cn
    return loss.sum(axis=(1, 2, 3, 4)) / (num_masks * Ht * Wt) * scale


def naive_dice(z, tgt, smooth, num_masks, scale=1.0):
    L, B, C, H, W = z.shape
    Ht, Wt = tgt.shape[1:]
    p = special.expit(upsample(z, Ht // H))
    y = np.stack([(tgt == c) for c in range(C)], axis=1).astype(np.float64)[None]
    I = (p * y).sum(axis=(3, 4))
    P = p.sum(axis=(3, 4))
    T = np.broadcast_to(y.sum(axis=(3, 4)), I.shape)
    d = (2 * I + smooth) / (P + T + smooth)
    return (1 - d).sum(axis=(1, 2)) / num_masks * scale, I, P, T


def case(seed, L=2, B=2, C=4, H=3, W=4, s=2, sigma=2.0):
    rng = np.random.default_rng(seed)
    z = rng.normal(0, sigma, size=(L, B, C, H, W))
    tgt = rng.integers(-1, C + 2, size=(B, H * s, W * s))  # includes out-of-range labels
    return z, tgt


def test_gt_total_rule():
    assert O.gt_total_from_targets(np.array([[[0, 3], [1, 1]]])) == 4
    assert O.gt_total_from_targets(np.zeros((1, 0, 2), dtype=np.int64)) == 0
    assert O.gt_total_from_targets(-np.ones((1, 2, 2), dtype=np.int64)) == 0


@pytest.mark.parametrize("s,bg,gamma,alpha,ug,normalize", [
    (1, -1, 0.0, -1.0, 1.0, True), (2, 0, 2.0, 0.25, 1.0, True), (3, 2, 0.0, -1.0, 0.0, False),
    (1, 5, 1.5, 0.6, 2.0, True)])
def test_pairwise_sigmoid_and_dice_vs_naive(s, bg, gamma, alpha, ug, normalize):
    rng = np.random.default_rng(7 + s)
    L, B, C, H, W = 1, 2, 5, 4, 3
    z = rng.normal(0, 2, size=(L, B, C, H, W))
    tgt = rng.integers(0, 4, size=(B, H * s, W * s))
    tgt[0, 0, 0] = 5  # GT slot 4 empty, slot 5 present: GT_total = 6
    tgt[tgt == 4] = 3
    G = int(tgt.max()) + 1
    rb, rd = naive_costs(z, tgt, G, bg, smooth=0.7, ss=1.3, ds=0.9, ug=ug, ugm=0.05,
                         gamma=gamma, alpha=alpha, normalize=normalize)
    b = O.pairwise_sigmoid_ce(z, tgt, bg, 1.3, gamma, alpha, ug, 0.05, normalize)
    d = O.pairwise_dice(z, tgt, 0.7, bg, 0.9, ug, 0.05)
    np.testing.assert_allclose(b, rb, rtol=1e-10)
    np.testing.assert_allclose(d, rd, rtol=1e-10)  # the naive dice uses no focal terms
    assert np.isinf(b).sum() > 0 and np.array_equal(np.isinf(b), np.isinf(d))


@pytest.mark.parametrize("s,gamma,alpha", [(1, 0.0, -1.0), (2, 2.0, 0.25), (3, 1.0, 0.7)])
def test_sigmoid_ce_vs_naive(s, gamma, alpha):
    z, tgt = case(11 + s, s=s)
    got = O.sigmoid_ce_loss(z, tgt, 3.0, 1.7, gamma, alpha)
    ref = naive_sigmoid_ce(z, tgt, 3.0, 1.7, gamma, alpha)
    np.testing.assert_allclose(got, ref, rtol=1e-11)


def test_sigmoid_ce_zero_closed_form():
    z, tgt = case(3)
    z[:] = 0.0
    L, B, C = z.shape[:3]
    got = O.sigmoid_ce_loss(z, tgt, 5.0, 2.0)
    np.testing.assert_allclose(got, np.full(L, B * C * math.log(2.0) * 2.0 / 5.0), rtol=1e-13)


@pytest.mark.parametrize("s,gamma,alpha", [(1, 0.0, -1.0), (2, 2.0, 0.25), (2, 0.5, 0.4)])
def test_sigmoid_ce_backward_fd(s, gamma, alpha):
    z, tgt = case(21 + s, L=1, B=1, C=3, H=2, W=3, s=s)
    g = np.array([1.3])
    got = O.sigmoid_ce_backward(g, z, tgt, 2.0, 0.8, gamma, alpha)
    h = 1e-6
    fd = np.zeros_like(z)
    for idx in np.ndindex(z.shape):
        zp, zm = z.copy(), z.copy()
        zp[idx] += h
        zm[idx] -= h
        fd[idx] = (g[0] * (naive_sigmoid_ce(zp, tgt, 2.0, 0.8, gamma, alpha)[0]
                           - naive_sigmoid_ce(zm, tgt, 2.0, 0.8, gamma, alpha)[0]) / (2 * h))
    np.testing.assert_allclose(got, fd, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("s", [1, 2, 4])
def test_dice_vs_naive(s):
    z, tgt = case(31 + s, s=s)
    loss, I, P, T = O.dice_loss(z, tgt, 0.5, 3.0, 1.4)
    rl, rI, rP, rT = naive_dice(z, tgt, 0.5, 3.0, 1.4)
    np.testing.assert_allclose(loss, rl, rtol=1e-12)
    np.testing.assert_allclose(I, rI, rtol=1e-12)
    np.testing.assert_allclose(P, rP, rtol=1e-12)
    np.testing.assert_allclose(T, rT, rtol=1e-12)


def test_dice_zero_closed_form():
    z, tgt = case(5, s=2)
    z[:] = 0.0
    L, B, C = z.shape[:3]
    Ht, Wt = tgt.shape[1:]
    loss, I, P, T = O.dice_loss(z, tgt, 1.0, 2.0)
    area = np.array([[(tgt[b] == c).sum() for c in range(C)] for b in range(B)], dtype=float)
    np.testing.assert_allclose(T[0], area)
    np.testing.assert_allclose(I[0], area / 2)
    np.testing.assert_allclose(P, np.full(P.shape, Ht * Wt / 2))
    dice = (area + 1.0) / (Ht * Wt / 2 + area + 1.0)
    np.testing.assert_allclose(loss, np.full(L, (1 - dice).sum() / 2.0), rtol=1e-13)


@pytest.mark.parametrize("s", [1, 2])
def test_dice_backward_fd(s):
    z, tgt = case(41 + s, L=1, B=1, C=3, H=2, W=3, s=s)
    g = np.array([0.9])
    _, I, P, T = O.dice_loss(z, tgt, 0.5, 2.0, 1.2)
    got = O.dice_loss_backward(g, z, tgt, I, P, T, 0.5, 2.0, 1.2)
    h = 1e-6
    fd = np.zeros_like(z)
    for idx in np.ndindex(z.shape):
        zp, zm = z.copy(), z.copy()
        zp[idx] += h
        zm[idx] -= h
        fd[idx] = g[0] * (naive_dice(zp, tgt, 0.5, 2.0, 1.2)[0][0]
                          - naive_dice(zm, tgt, 0.5, 2.0, 1.2)[0][0]) / (2 * h)
    np.testing.assert_allclose(got, fd, rtol=1e-6, atol=1e-10)
