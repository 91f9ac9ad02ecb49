"""GPU parity of the point-sampling front end against the float64 oracle
(oracle/points_oracle.py): bilinear point_sample (grid_sample semantics,
functions/utils.py:12-20), the labels under the points, and the point-sampled
pairwise sigmoid-CE / dice costs (functions/sigmoid/pw_sigmoid_ce.py:407-550,
functions/dice/pw_dice_loss.py:174-268) for given points, through the
`mask_loss` extension and its C ABI; plus the Python front-ends with their
own torch.rand draws, reproduced from the same seed.

Tolerances: sampled values |g - r| <= rtol (|r| + max|input|) with rtol 1e-5
for float32 (a bilinear value is a sum of four corner products, so float32
rounding scales with the corners' magnitude, not with the result's, which
cancels towards zero) and the output dtype's rounding (2^-8 bfloat16, 2^-10
float16) otherwise; costs as the north star (float32 1e-5, bfloat16 2e-2, float16
2e-3, floor 1e-2); labels bit-exact.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import points_oracle as PO  # noqa: E402

pytestmark = pytest.mark.gpu

TDT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}
SAMPLE_RTOL = {"float32": 1e-5, "bfloat16": 2.0 ** -8, "float16": 2.0 ** -10}
COST_RTOL = {"float32": 1e-5, "bfloat16": 2e-2, "float16": 2e-3}


@pytest.fixture(scope="module")
def ml():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mask_loss_amd
    return mask_loss_amd.mask_loss


def close(g, r, rtol, floor):
    g = np.asarray(g, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    assert np.array_equal(np.isinf(g), np.isinf(r)), "inf pattern differs"
    f = np.isfinite(r)
    err = np.abs(g[f] - r[f])
    bound = rtol * (np.abs(r[f]) + floor)
    assert not (err > bound).any(), f"max err {err.max():.3e}, worst ratio {(err / bound).max():.3f}"


def as_dtype(x, dt):
    """numpy float64 -> values representable in `dt` (float64 copy) and the device tensor"""
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(TDT[dt])
    return t.double().numpy(), t.cuda()


def coords_with_edges(rng, N, P, lo=-0.2, hi=1.2):
    c = rng.uniform(lo, hi, size=(N, P, 2)).astype(np.float32)
    c[:, :6] = np.array([[0, 0], [1, 1], [0.5, 0.5], [1, 0], [0, 1], [np.nan, 0.3]], np.float32)
    return c


@pytest.mark.parametrize("dt", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("align", [False, True])
@pytest.mark.parametrize("H,W", [(9, 13), (130, 140), (256, 257)])
def test_point_sample(ml, dt, align, H, W):
    # planes of up to 64 KB are staged in LDS (several per workgroup when they
    # fit), larger ones are gathered from memory: (130, 140) float32 and
    # (256, 257) in every dtype take the second path
    rng = np.random.default_rng(7 + align + H)
    x64, x = as_dtype(rng.normal(0, 2, size=(3, 5, H, W)), dt)
    c = coords_with_edges(rng, 3, 517)
    got = ml.point_sample(x, torch.from_numpy(c).cuda(), align)
    assert got.dtype == TDT[dt] and got.shape == (3, 5, 517)
    ref = PO.point_sample(x64, c, align)
    close(got.double().cpu().numpy(), ref, SAMPLE_RTOL[dt], np.abs(x64).max())


def test_point_sample_grid_and_wrapper(ml):
    from mask_loss_amd.functions import point_sample
    rng = np.random.default_rng(3)
    x64, x = as_dtype(rng.normal(0, 2, size=(2, 4, 16, 8)), "float32")
    c = rng.uniform(0, 1, size=(2, 5, 7, 2)).astype(np.float32)
    got = point_sample(x, torch.from_numpy(c).cuda().double(), align_corners=True)
    assert got.shape == (2, 4, 5, 7)
    close(got.cpu().numpy(), PO.point_sample(x64, c, True), 1e-5, np.abs(x64).max())
    with pytest.raises(NotImplementedError):
        point_sample(x, torch.from_numpy(c).cuda(), mode="nearest")


def test_point_sample_masks(ml):
    rng = np.random.default_rng(11)
    L, B, Q, H, W, P = 2, 3, 7, 10, 12, 300
    z64, z = as_dtype(rng.normal(0, 3, size=(L, B, Q, H, W)), "bfloat16")
    c = coords_with_edges(rng, B, P, 0.0, 1.0)
    got = ml.point_sample_masks(z, torch.from_numpy(c).cuda(), False).double().cpu().numpy()
    assert got.shape == (L, B, Q, P)
    for b in range(B):
        ref = PO.point_sample(z64[:, b].reshape(L * Q, 1, H, W), np.repeat(c[b:b + 1], L * Q, 0))
        close(got[:, b], ref[:, 0].reshape(L, Q, P), SAMPLE_RTOL["bfloat16"], 1e-2 * np.abs(z64).max())


@pytest.mark.parametrize("Ht,Wt", [(64, 48), (1, 7), (5, 1)])
def test_point_labels(ml, Ht, Wt):
    rng = np.random.default_rng(Ht + Wt)
    t = rng.integers(-1, 30, size=(4, Ht, Wt)).astype(np.int64)
    c = coords_with_edges(rng, 4, 1000)
    got = ml.point_labels(torch.from_numpy(t).cuda(), torch.from_numpy(c).cuda()).cpu().numpy()
    np.testing.assert_array_equal(got, PO.point_labels(t, c))


def sampling_case(seed, L=2, B=3, C=20, h=16, w=12, Ht=64, Wt=48, G=9, P=1000):
    rng = np.random.default_rng(seed)
    z = rng.normal(0, 2, size=(L, B, C, h, w))
    t = rng.integers(0, G + 1, size=(B, Ht, Wt)).astype(np.int64)
    t[1] = np.where(t[1] == 3, 0, t[1])  # class 3 absent from image 1
    t[2] = np.where(t[2] == G, 1, t[2])
    t[2, 0, 0] = G                       # present at one pixel (rarely at a point)
    t[0] = 0                             # image 0: background only
    c = rng.uniform(0, 1, size=(B, P, 2)).astype(np.float32)
    return z, t, c


@pytest.mark.parametrize("dt", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("bg", [-1, 0])
def test_sampling_costs(ml, dt, bg):
    z, t, c = sampling_case(5 + bg)
    z64, zt = as_dtype(z, dt)
    tt, ct = torch.from_numpy(t).cuda(), torch.from_numpy(c).cuda()
    bce = ml.forward_pw_sigmoid_ce_loss_sampling(zt, tt, ct, bg, 1.5, 0.0, -1.0, False)
    dice = ml.forward_pw_dice_loss_sampling(zt, tt, ct, 1.0, bg, 2.0, False)
    bgo = None if bg < 0 else bg
    rb = PO.pairwise_sigmoid_ce_sampling(z64, t, c, background_index=bgo, scale=1.5)
    rd = PO.pairwise_dice_sampling(z64, t, c, smooth=1.0, background_index=bgo, scale=2.0)
    assert bce.shape == rb.shape and dice.shape == rd.shape
    close(bce.cpu().numpy(), rb, COST_RTOL[dt], 1e-2)
    close(dice.cpu().numpy(), rd, COST_RTOL[dt], 1e-2)


@pytest.mark.parametrize("gamma,alpha,align", [(2.0, 0.25, False), (1.5, -1.0, True)])
def test_sampling_costs_focal_align(ml, gamma, alpha, align):
    z, t, c = sampling_case(21, C=7, P=333)
    z64, zt = as_dtype(z, "float32")
    tt, ct = torch.from_numpy(t).cuda(), torch.from_numpy(c).cuda()
    bce = ml.forward_pw_sigmoid_ce_loss_sampling(zt, tt, ct, 0, 1.0, gamma, alpha, align)
    rb = PO.pairwise_sigmoid_ce_sampling(z64, t, c, background_index=0, gamma=gamma,
                                         alpha=None if alpha < 0 else alpha, align_corners=align)
    close(bce.cpu().numpy(), rb, 1e-5, 1e-2)
    dice = ml.forward_pw_dice_loss_sampling(zt, tt, ct, 0.5, 0, 1.0, align)
    rd = PO.pairwise_dice_sampling(z64, t, c, smooth=0.5, background_index=0, align_corners=align)
    close(dice.cpu().numpy(), rd, 1e-5, 1e-2)


def test_sampling_wrappers_draw_like_the_reference(ml):
    from mask_loss_amd.functions import (pairwise_dice_loss_sampling_py,
                                         pairwise_sigmoid_cross_entropy_loss_sampling_py)
    z, t, _ = sampling_case(8, C=5, P=10)
    z64, zt = as_dtype(z, "bfloat16")
    tt = torch.from_numpy(t).cuda()
    torch.manual_seed(1234)
    got = pairwise_sigmoid_cross_entropy_loss_sampling_py(zt, tt, background_index=0, num_points=700)
    gd = pairwise_dice_loss_sampling_py(zt, tt, smooth=1.0, background_index=0, num_points=700)
    assert got.dtype == torch.bfloat16 and got.shape == (2, 3, 5, int(t.max()))
    # the reference's draws: torch.rand(1, P, 2) per image in order, except for
    # image 0, which holds only the background (pw_sigmoid_ce.py:480-486)
    torch.manual_seed(1234)

    def draws():
        r = [torch.rand(1, 700, 2, device="cuda") for _ in range(2)]
        return torch.cat([torch.zeros(1, 700, 2, device="cuda")] + r).cpu().numpy()

    c1 = draws()
    c2 = draws()
    # and then the generator stands where the reference's leaves it
    nxt = torch.rand(1, device="cuda").item()
    torch.manual_seed(1234)
    pairwise_sigmoid_cross_entropy_loss_sampling_py(zt, tt, background_index=0, num_points=700)
    pairwise_dice_loss_sampling_py(zt, tt, smooth=1.0, background_index=0, num_points=700)
    assert torch.rand(1, device="cuda").item() == nxt
    rb = PO.pairwise_sigmoid_ce_sampling(z64, t, c1, background_index=0)
    rd = PO.pairwise_dice_sampling(z64, t, c2, background_index=0)
    close(got.double().cpu().numpy(), rb, 2e-2, 1e-2)
    close(gd.double().cpu().numpy(), rd, 2e-2, 1e-2)


def test_uncertain_point_coords(ml):
    from mask_loss_amd.functions import calculate_uncertainty, get_uncertain_point_coords_with_randomness
    rng = np.random.default_rng(2)
    x64, x = as_dtype(rng.normal(0, 2, size=(4, 1, 20, 24)), "float32")
    torch.manual_seed(99)
    got = get_uncertain_point_coords_with_randomness(x, calculate_uncertainty, 120, 3, 0.75)
    assert got.shape == (4, 120, 2)
    got = got.cpu().numpy()
    torch.manual_seed(99)
    over = torch.rand(4, 360, 2, device="cuda").cpu().numpy()
    rand_tail = torch.rand(4, 30, 2, device="cuda").cpu().numpy()
    unc = -np.abs(PO.point_sample(x64, over)[:, 0, :])  # (4, 360)
    for n in range(4):
        order = np.sort(unc[n])[::-1]
        kth, nxt = order[89], order[90]
        picked = [int(np.flatnonzero((over[n] == p).all(axis=1))[0]) for p in got[n, :90]]
        assert len(set(picked)) == 90
        # every pick is among the 90 most uncertain (up to float32 rounding at the boundary)
        assert all(unc[n][i] >= min(kth, nxt) - 1e-5 for i in picked)
        np.testing.assert_array_equal(got[n, 90:], rand_tail[n])


def test_validation(ml):
    x = torch.zeros(2, 3, 4, 4, device="cuda")
    c = torch.zeros(2, 5, 2, device="cuda")
    with pytest.raises(RuntimeError, match="float32"):
        ml.point_sample(x, c.double(), False)
    with pytest.raises(RuntimeError, match="batch size"):
        ml.point_sample(x, torch.zeros(3, 5, 2, device="cuda"), False)
    with pytest.raises(RuntimeError):
        ml.point_sample(x.cpu(), c.cpu(), False)
    z = torch.zeros(1, 2, 3, 4, 4, device="cuda")
    t = torch.zeros(2, 8, 8, dtype=torch.long, device="cuda")
    with pytest.raises(RuntimeError, match="num_points"):
        ml.forward_pw_dice_loss_sampling(z, t, torch.zeros(2, 0, 2, device="cuda"), 1.0, -1, 1.0, False)
    # background only: no GT columns
    out = ml.forward_pw_sigmoid_ce_loss_sampling(z, t, c, 0, 1.0, 0.0, -1.0, False)
    assert out.shape == (1, 2, 3, 0)


@pytest.mark.parametrize("dt", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("H,W,P,C", [
    (9, 13, 777, 5), (130, 140, 777, 5), (9, 13, 17000, 5), (130, 140, 17000, 5),
    (9, 13, 777, 9), (37, 29, 1025, 8), (128, 128, 12544, 8), (9, 13, 16384, 8), (130, 140, 777, 9)])
def test_point_sample_backward(ml, dt, H, W, P, C):
    # C = 5 planes per coordinate set: float atomics in LDS for the (9, 13)
    # plane and into a float workspace for the 72.8 KB (130, 140) plane;
    # P = 17000 gives up to a few hundred samples per cell of the small plane.
    # C >= 8 with at most 16,384 cells and points: the corner entries grouped
    # by cell and gathered per plane (128 x 128 at configuration 2's 12,544
    # points: eight rounds of 2048 cells, each with its ~6,300 entries staged
    # in LDS; (9, 13) with 16,384 points: one round of ~65,000 entries, too
    # many to stage, read from memory); (130, 140) stays on the float
    # workspace.
    rng = np.random.default_rng(31 + H + P + C)
    c = coords_with_edges(rng, 3, P)
    g64, g = as_dtype(rng.normal(0, 1, size=(3, C, P)), dt)
    g64[1, 2] = 0.0  # an all-zero row (an unmatched query)
    g[1, 2] = 0
    got = ml.point_sample_backward(g, torch.from_numpy(c).cuda(), H, W, False)
    assert got.dtype == TDT[dt] and got.shape == (3, C, H, W)
    ref = PO.point_sample_backward(g64, c, H, W, False)
    assert (got[1, 2] == 0).all()
    # float32 sums in another order: a few ulps of the cell's largest partial sum
    close(got.double().cpu().numpy(), ref, SAMPLE_RTOL[dt], np.abs(ref).max())


@pytest.mark.parametrize("H,W,P,C", [(37, 29, 1025, 8), (128, 128, 12544, 8), (9, 13, 777, 9)])
def test_point_sample_backward_align_corners(ml, H, W, P, C):
    """align_corners=True on the grouped path (C >= 8 planes per coordinate
    set: corner entries bucketed by base cell, then gathered per plane), with
    coordinates outside [0, 1] (coords_with_edges), against the oracle's
    adjoint of grid_sample with align_corners=True."""
    rng = np.random.default_rng(57 + H + P + C)
    c = coords_with_edges(rng, 3, P)
    g64, g = as_dtype(rng.normal(0, 1, size=(3, C, P)), "float32")
    g64[2, 1] = 0.0  # an all-zero row (an unmatched query)
    g[2, 1] = 0
    got = ml.point_sample_backward(g, torch.from_numpy(c).cuda(), H, W, True)
    ref = PO.point_sample_backward(g64, c, H, W, True)
    assert (got[2, 1] == 0).all()
    close(got.double().cpu().numpy(), ref, SAMPLE_RTOL["float32"], np.abs(ref).max())


def test_point_sample_autograd_4d_grid(ml):
    from mask_loss_amd.functions import point_sample
    rng = np.random.default_rng(4)
    x64, x = as_dtype(rng.normal(0, 2, size=(2, 3, 11, 6)), "float32")
    x.requires_grad_(True)
    c = rng.uniform(-0.1, 1.1, size=(2, 4, 5, 2)).astype(np.float32)
    out = point_sample(x, torch.from_numpy(c).cuda(), align_corners=True)
    g = rng.normal(size=out.shape)
    out.backward(torch.from_numpy(g).float().cuda())
    ref = PO.point_sample_backward(g, c, 11, 6, True)
    close(x.grad.double().cpu().numpy(), ref, 1e-5, np.abs(ref).max())
    with pytest.raises(NotImplementedError, match="coordinates"):
        point_sample(x, torch.from_numpy(c).cuda().requires_grad_(True))


def test_point_sampled_matching_step_gradient_reaches_dense_logits(ml):
    """Mask2Former-style step: dense logits sampled at the points, the fused
    cost -> assignment -> loss on the 1 x P map of sampled logits and point
    labels, backward through the sampling to the dense logits."""
    from mask_loss_amd.functions import MaskMatchingFunction, point_sample
    from oracle import mask_oracle as O
    rng = np.random.default_rng(9)
    B, Q, h, w, P, C = 2, 24, 16, 12, 600, 7
    z = rng.normal(0, 2, size=(1, B, Q, h, w)).astype(np.float32)
    t = np.zeros((B, 64, 48), np.int64)
    for b in range(B):
        for g in range(1, 6):
            y0, x0 = rng.integers(0, 40), rng.integers(0, 30)
            t[b, y0:y0 + 20, x0:x0 + 16] = g
    cls_t = np.full((B, 6), -1, np.int64)
    cls_t[:, 1:] = rng.integers(0, C - 1, size=(B, 5))
    zc = rng.normal(0, 1, size=(1, B, Q, C)).astype(np.float32)
    c = rng.uniform(0, 1, size=(B, P, 2)).astype(np.float32)
    zt = torch.from_numpy(z).cuda().requires_grad_(True)
    ct = torch.from_numpy(c).cuda()
    lab = ml.point_labels(torch.from_numpy(t).cuda(), ct).view(B, 1, P)
    zs = point_sample(zt.view(B, Q, h, w), ct).view(1, B, Q, 1, P)
    zct = torch.from_numpy(zc).cuda()
    ctt = torch.from_numpy(cls_t).cuda()
    p2g, pr, m, d, cl = MaskMatchingFunction.apply(
        zs, lab, zct, ctt, 1.0, 1.0, 1.0, 1.0, 0, 1.0, 0.05, True, 1e30, -1.0, True, False, 1,
        "global", 0.0, None, 0.0, None, C - 1, "softmax")
    (m.sum() + d.sum() + cl.sum()).backward()
    assert int((p2g >= 0).sum()) > 0
    # oracle: the same chain in float64 with the GPU's assignment
    zs64 = PO.point_sample(z[0].astype(np.float64), c)[None, :, :, None, :]
    lab64 = PO.point_labels(t, c)[:, None, :]
    gzs, _ = O.matching_backward(np.ones(1), np.ones(1), np.ones(1), zs64, lab64,
                                 zc.astype(np.float64), cls_t, p2g.cpu().numpy(),
                                 background_index=0, force_cls=True, void_class_index=C - 1,
                                 use_softmax=True)
    ref = PO.point_sample_backward(gzs[0, :, :, 0, :], c, h, w)[None]
    close(zt.grad.double().cpu().numpy(), ref, 1e-5, np.abs(ref).max())


@pytest.mark.parametrize("dt", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("P", [1025, 12544])
@pytest.mark.parametrize("H,W", [(32, 32), (37, 29)])
def test_point_sample_many_points(ml, dt, P, H, W):
    """More points than the gather's 1024-thread workgroup: its point loop
    takes several rounds (12,544 is configuration 2's count).  32 x 32 planes
    are staged several per workgroup; 37 x 29 planes are not a multiple of the
    16-byte staging loads."""
    rng = np.random.default_rng(P + H)
    x64, x = as_dtype(rng.normal(0, 2, size=(2, 6, H, W)), dt)
    c = coords_with_edges(rng, 2, P)
    got = ml.point_sample(x, torch.from_numpy(c).cuda(), False)
    assert got.dtype == TDT[dt] and got.shape == (2, 6, P)
    ref = PO.point_sample(x64, c, False)
    close(got.double().cpu().numpy(), ref, SAMPLE_RTOL[dt], np.abs(x64).max())
