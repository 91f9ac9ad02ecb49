"""The forward-only autograd front-ends with the reference's names and
signatures, run on the GPU: PairwiseMaskLossFunction (reference
functions/mask/pw_mask.py:21-115), PairwiseSigmoidCELossFunction and
PairwiseDiceLossFunction (functions/sigmoid/pw_sigmoid_ce.py:15-57,
functions/dice/pw_dice_loss.py:15-57), PairwiseSigmoidLabelLossFunction and
PairwiseSoftmaxLabelLossFunction / pairwise_softmax_label_loss
(functions/label/*.py).

Each wrapper's output is compared with the float64 oracle (north-star
tolerances: float32 rel 1e-5, bfloat16 2e-2, float16 2e-3, as
|g - r| <= rtol (|r| + 1e-2)), and with the extension call it forwards to, bit
for bit, so that default-argument handling (None -> the reference's defaults)
is what is being checked.  Validation messages follow the reference's."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import mask_oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu

RTOL = {"float32": 1e-5, "bfloat16": 2e-2, "float16": 2e-3}
TDT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


@pytest.fixture(scope="module")
def F():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mask_loss_amd.functions as F
    return F


@pytest.fixture(scope="module")
def ml():
    import mask_loss_amd
    return mask_loss_amd.mask_loss


def close(g, r, rtol, floor=1e-2):
    g = np.asarray(g, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    assert np.array_equal(np.isinf(g), np.isinf(r)), "inf pattern differs"
    f = np.isfinite(r)
    err = np.abs(g[f] - r[f])
    bound = rtol * (np.abs(r[f]) + floor)
    assert not (err > bound).any(), f"max err {err.max():.3e}, worst ratio {(err / bound).max():.3f}"


def inputs(seed, L=1, B=2, Q=24, H=16, W=16, G=6, C=9, dtype="float32", sigma=2.0):
    rng = np.random.default_rng(seed)
    z = rng.normal(0, sigma, size=(L, B, Q, H, W)).astype(np.float32)
    zt = torch.from_numpy(z).to(TDT[dtype])
    z64 = zt.float().numpy().astype(np.float64)  # the values the kernels see
    tgt = np.zeros((B, H, W), np.int64)
    yy, xx = np.mgrid[0:H, 0:W]
    for b in range(B):
        for g in range(1, G + 1):
            cy, cx, r = rng.uniform(0, H), rng.uniform(0, W), rng.uniform(1, H / 3)
            tgt[b][(yy - cy) ** 2 + (xx - cx) ** 2 <= r * r] = g
    ct = np.full((B, G + 2), -1, np.int64)
    ct[:, 1:G + 1] = rng.integers(0, C - 1, size=(B, G))
    zc = rng.normal(0, 1, size=(L, B, Q, C)).astype(np.float32)
    return dict(z=zt.cuda(), z64=z64, tgt=torch.from_numpy(tgt).cuda(), tgt_np=tgt,
                zc=torch.from_numpy(zc).cuda(), zc64=zc.astype(np.float64),
                ct=torch.from_numpy(ct).cuda(), ct_np=ct, dtype=dtype)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("label_loss", ["sigmoid", "softmax"])
def test_pairwise_mask_loss_function(F, ml, dtype, label_loss):
    x = inputs(11, dtype=dtype, sigma=3.0 if dtype == "bfloat16" else 2.0)
    # None arguments take the reference's defaults (smooth 1, scales 1,
    # background -1, uncertainty 1 / 0.05, no focal terms, normalized)
    got = F.PairwiseMaskLossFunction.apply(x["z"], x["tgt"], x["zc"], x["ct"], None, None, None, None,
                                           0, None, None, None, None, None, None, None, label_loss)
    soft = label_loss == "softmax"
    direct = ml.pairwise_mask_loss_forward(x["z"], x["tgt"], x["zc"], x["ct"], 1.0, 1.0, 1.0, 1.0, 0,
                                           1.0, 0.05, 0.0, -1.0, 0.0, -1.0, soft, True)
    assert torch.equal(got, direct)
    ref = O.pairwise_mask_loss_forward(x["z64"], x["tgt_np"], x["zc64"], x["ct_np"], 1.0, 1.0, 1.0, 1.0,
                                       0, 1.0, 0.05, 0.0, -1.0, 0.0, -1.0, soft, True)
    g = got.cpu().numpy()
    close(g[0], ref[0], RTOL[dtype])
    close(g[1], ref[1], RTOL[dtype])
    close(g[2], ref[2], 1e-5)


def test_pairwise_mask_loss_function_focal_scales(F):
    x = inputs(12, Q=20, G=5)
    got = F.PairwiseMaskLossFunction.apply(x["z"], x["tgt"], x["zc"], x["ct"], 0.5, 1.3, 0.7, 2.0, 0,
                                           2.0, 0.1, False, 2.0, 0.25, 1.5, 0.6, "sigmoid")
    ref = O.pairwise_mask_loss_forward(x["z64"], x["tgt_np"], x["zc64"], x["ct_np"], 0.5, 1.3, 0.7, 2.0,
                                       0, 2.0, 0.1, 2.0, 0.25, 1.5, 0.6, False, False)
    g = got.cpu().numpy()
    for i in range(3):
        close(g[i], ref[i], 1e-5)


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_pairwise_sigmoid_ce_function(F, dtype):
    x = inputs(13, Q=7, dtype=dtype)
    z5 = x["z"]  # (L, B, C, h, w): the query axis plays the channel axis
    got = F.PairwiseSigmoidCELossFunction.apply(z5, x["tgt"], None, None, None, None)
    ref = O.pairwise_sigmoid_ce(x["z64"], x["tgt_np"], -1, 1.0, 0.0, -1.0, 1.0, 0.05, True)
    close(got.float().cpu().numpy(), ref, RTOL[dtype])
    got2 = F.PairwiseSigmoidCELossFunction.apply(z5, x["tgt"], 0, 1.3, 2.0, 0.25, 2.0, 0.1, False)
    ref2 = O.pairwise_sigmoid_ce(x["z64"], x["tgt_np"], 0, 1.3, 2.0, 0.25, 2.0, 0.1, False)
    close(got2.float().cpu().numpy(), ref2, RTOL[dtype])


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_pairwise_dice_function(F, dtype):
    x = inputs(14, Q=7, dtype=dtype, sigma=3.0 if dtype == "bfloat16" else 2.0)
    got = F.PairwiseDiceLossFunction.apply(x["z"], x["tgt"], None, None, None)
    ref = O.pairwise_dice(x["z64"], x["tgt_np"], 1.0, -1, 1.0, 1.0, 0.05)
    close(got.float().cpu().numpy(), ref, RTOL[dtype])
    got2 = F.PairwiseDiceLossFunction.apply(x["z"], x["tgt"], 0.5, 0, 0.9, 2.0, 0.1)
    ref2 = O.pairwise_dice(x["z64"], x["tgt_np"], 0.5, 0, 0.9, 2.0, 0.1)
    close(got2.float().cpu().numpy(), ref2, RTOL[dtype])


def test_label_loss_functions(F, ml):
    x = inputs(15, Q=30, C=17)
    got = F.PairwiseSigmoidLabelLossFunction.apply(x["zc"], x["ct"])
    ref = O.pairwise_sigmoid_label_cost(x["zc64"], x["ct_np"], -1, 1.0, 0.0, -1.0)
    close(got.cpu().numpy(), ref, 1e-5)
    got = F.PairwiseSigmoidLabelLossFunction.apply(x["zc"], x["ct"], 0, 1.7, 2.0, 0.25)
    assert torch.equal(got, ml.forward_pw_sigmoid_label_loss(x["zc"], x["ct"], 0, 1.7, 2.0, 0.25))
    ref = O.pairwise_sigmoid_label_cost(x["zc64"], x["ct_np"], 0, 1.7, 2.0, 0.25)
    close(got.cpu().numpy(), ref, 1e-5)

    got = F.PairwiseSoftmaxLabelLossFunction.apply(x["zc"], x["ct"])
    ref = O.pairwise_softmax_label_cost(x["zc64"], x["ct_np"], -1, 1.0)
    close(got.cpu().numpy(), ref, 1e-5)
    got = F.pairwise_softmax_label_loss(x["zc"], x["ct"], background_index=0, scale=1.7)
    assert torch.equal(got, ml.forward_pw_softmax_label_loss(x["zc"], x["ct"], 0, 1.7))
    ref = O.pairwise_softmax_label_cost(x["zc64"], x["ct_np"], 0, 1.7)
    close(got.cpu().numpy(), ref, 1e-5)


def test_wrapper_validation(F):
    x = inputs(16, Q=6)
    with pytest.raises(ValueError, match="focal_gamma must be non-negative"):
        F.PairwiseSigmoidLabelLossFunction.apply(x["zc"], x["ct"], None, 1.0, -1.0, None)
    with pytest.raises(ValueError, match="focal_alpha must be in"):
        F.PairwiseSigmoidLabelLossFunction.apply(x["zc"], x["ct"], None, 1.0, 0.0, 1.5)
    with pytest.raises(AssertionError, match="Batch size mismatch"):
        F.PairwiseMaskLossFunction.apply(x["z"], x["tgt"][:1], x["zc"], x["ct"], None, None, None,
                                         None, 0, None, None, None, None, None, None, None, "sigmoid")
    with pytest.raises(AssertionError, match="Batch size mismatch"):
        F.PairwiseDiceLossFunction.apply(x["z"], x["tgt"][:1], None, None, None)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_losses_dispatchers(F, dtype):
    """functions/losses.py:8-67: (B, C, h, w) logits give a scalar, (L, B, C,
    h, w) one loss per layer; both against the float64 oracle."""
    x = inputs(31, L=2, B=2, Q=12, H=8, W=8, G=5, dtype=dtype)
    B, C = 2, 12
    z4 = x["z"][0]
    tg = torch.from_numpy(np.kron(x["tgt_np"], np.ones((1, 2, 2), np.int64))).cuda()  # s = 2
    ce = F.sigmoid_cross_entropy_loss(z4, tg, scale=1.5)
    dl = F.dice_loss(z4, tg, smooth=1.0, scale=0.7)
    assert ce.dim() == 0 and dl.dim() == 0
    tgn = tg.cpu().numpy()
    close(ce.item(), O.sigmoid_ce_loss(x["z64"][:1], tgn, B * C, scale=1.5)[0], RTOL[dtype])
    close(dl.item(), O.dice_loss(x["z64"][:1], tgn, 1.0, B * C, scale=0.7)[0][0], RTOL[dtype])
    ce5 = F.sigmoid_cross_entropy_loss(x["z"], tg, num_masks=10.0)
    dl5 = F.dice_loss(x["z"], tg, num_masks=10.0)
    assert tuple(ce5.shape) == (2,) and tuple(dl5.shape) == (2,)
    close(ce5.cpu().numpy(), O.sigmoid_ce_loss(x["z64"], tgn, 10.0), RTOL[dtype])
    close(dl5.cpu().numpy(), O.dice_loss(x["z64"], tgn, 1e-6, 10.0)[0], RTOL[dtype])


def test_losses_dispatcher_errors(F):
    x = inputs(32, L=1, B=2, Q=4, H=8, W=8, G=3)
    z4 = x["z"][0]
    cm = torch.arange(256, device=z4.device)
    for fn in (F.sigmoid_cross_entropy_loss, F.dice_loss):
        with pytest.raises(NotImplementedError, match="multi-class"):
            fn(z4, x["tgt"], class_mapping=cm)
        with pytest.raises(NotImplementedError, match="pure-PyTorch"):
            fn(z4, x["tgt"], implementation="python")
        # every value other than "python" runs the GPU operator
        # (functions/losses.py:24-33, 57-67)
        a = fn(z4, x["tgt"], num_masks=3.0, implementation="triton")
        b = fn(z4, x["tgt"], num_masks=3.0)
        assert torch.equal(a, b)
        with pytest.raises(ValueError, match="logits must be"):
            fn(z4[0], x["tgt"])
