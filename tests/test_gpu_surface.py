"""GPU parity of the standalone operators against the float64 oracle:
forward_pw_sigmoid_ce_loss, forward_pw_dice_loss (pairwise costs with GT
slots 0..max(targets)) and forward/backward_sigmoid_ce_loss,
forward/backward_dice_loss (per-class losses over dense class logits), through
the `mask_loss` extension and its C ABI, plus the autograd front-ends.

Tolerances (north star): float32 logits rel 1e-5, bfloat16 2e-2, float16
2e-3, as |g - r| <= rtol (|r| + floor) with floor 1e-2 for costs and losses
and 1e-2 max|r| for gradients.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import mask_oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu

RTOL = {"float32": 1e-5, "bfloat16": 2e-2, "float16": 2e-3}
# gradients are returned in the logits' dtype: half of float16's subnormal
# spacing (2^-24) is the least error a float16 result can carry below 2^-14
STORE = {"float32": 0.0, "bfloat16": 0.0, "float16": 2.0 ** -25}
TDT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


@pytest.fixture(scope="module")
def ml():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mask_loss_amd
    return mask_loss_amd.mask_loss


def close(g, r, rtol, floor, extra=None):
    """|g - r| <= rtol (|r| + floor) (+ extra, an elementwise absolute term)."""
    g = np.asarray(g, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    assert np.array_equal(np.isinf(g), np.isinf(r)), "inf pattern differs"
    f = np.isfinite(r)
    err = np.abs(g[f] - r[f])
    bound = rtol * (np.abs(r[f]) + floor)
    if extra is not None:
        bound = bound + np.broadcast_to(extra, r.shape)[f]
    assert not (err > bound).any(), f"max err {err.max():.3e}, worst ratio {(err / bound).max():.3f}"


def dice_grad_cancellation(grad_out, z64, tgt, I, P, T, smooth, num_masks, scale):
    """Absolute rounding error that float32 arithmetic (the reference's too)
    incurs in the dice gradient's difference 2 n D - N2 (2 I + smooth), which
    cancels for partial counts: 8 ulps of the larger product, carried through
    the gradient's other factors."""
    L, B, C, H, W = z64.shape
    N2 = float((tgt.shape[1] // H) ** 2)
    n = O.label_counts(tgt, H, W, C).astype(np.float64).reshape(1, B, C, H, W)
    p = 1.0 / (1.0 + np.exp(-z64))
    D = (np.asarray(P, np.float64) + np.asarray(T, np.float64) + smooth)[..., None, None]
    num = (2.0 * np.asarray(I, np.float64) + smooth)[..., None, None]
    mag = np.maximum(2.0 * n * D, N2 * num)
    coef = np.abs(np.asarray(grad_out, np.float64)).reshape(L, 1, 1, 1, 1) / num_masks * scale
    return 8 * 2.0 ** -24 * mag / (D * D) * p * (1 - p) * coef


def make(seed, L=1, B=2, C=5, H=16, W=16, s=1, dtype="float32", sigma=2.0, labels=None,
         extreme=False):
    rng = np.random.default_rng(seed)
    z = rng.normal(0, sigma, size=(L, B, C, H, W)).astype(np.float32)
    if extreme:
        z.reshape(-1)[rng.choice(z.size, size=20, replace=False)] = rng.choice(
            np.array([64.0, -70.0, 300.0, -1000.0], np.float32), size=20)
    hi = labels if labels is not None else C
    tgt = rng.integers(-1, hi + 1, size=(B, H * s, W * s)).astype(np.int64)
    # blobs so that counts are not uniform noise
    yy, xx = np.mgrid[0:H * s, 0:W * s]
    for b in range(B):
        for g in range(min(hi, 4)):
            cy, cx = rng.uniform(0, H * s), rng.uniform(0, W * s)
            r = rng.uniform(1, H * s / 3)
            tgt[b][(yy - cy) ** 2 + (xx - cx) ** 2 <= r * r] = g
    zt = torch.from_numpy(z).to(TDT[dtype])
    return dict(z=zt.cuda(), z64=zt.float().numpy().astype(np.float64), tgt=torch.from_numpy(tgt).cuda(),
                tgt_np=tgt, dtype=dtype)


PW_CASES = [
    dict(name="f32", kw={}, p={}),
    dict(name="bf16", kw=dict(dtype="bfloat16", sigma=3.0), p={}),
    dict(name="f16", kw=dict(dtype="float16"), p={}),
    dict(name="f32_s2_bg0_focal", kw=dict(s=2, H=8, W=8), p=dict(bg=0, gamma=2.0, alpha=0.25)),
    dict(name="f32_s4_nonorm_ug0", kw=dict(s=4, H=8, W=8), p=dict(ug=0.0, normalize=False)),
    # 16-bit counts (the reference's uint8 counts overflow from s = 16 on)
    dict(name="f32_s16_u16_counts", kw=dict(s=16, H=4, W=4), p=dict(bg=0)),
    dict(name="bf16_s17_split_counts", kw=dict(s=17, H=3, W=5, dtype="bfloat16", sigma=3.0), p={}),
    dict(name="f32_bg_mid_ug2", kw=dict(C=7, H=9, W=7), p=dict(bg=2, ug=2.0, ug_min=0.1)),
    dict(name="f32_many_gt", kw=dict(C=3, H=32, W=32, labels=60), p=dict(bg=0)),
    dict(name="bf16_extreme", kw=dict(dtype="bfloat16", sigma=3.0, extreme=True, H=32, W=32), p={}),
]


def pw_params(p):
    d = dict(bg=-1, gamma=0.0, alpha=-1.0, ug=1.0, ug_min=0.05, normalize=True, scale=1.3,
             smooth=0.7, dscale=0.9)
    d.update(p)
    return d


@pytest.mark.parametrize("case", PW_CASES, ids=lambda c: c["name"])
def test_pairwise_sigmoid_ce(ml, case):
    x = make(5, **case["kw"])
    P = pw_params(case["p"])
    got = ml.forward_pw_sigmoid_ce_loss(x["z"], x["tgt"], P["bg"], P["scale"], P["gamma"],
                                        P["alpha"], P["ug"], P["ug_min"], P["normalize"])
    ref = O.pairwise_sigmoid_ce(x["z64"], x["tgt_np"], P["bg"], P["scale"], P["gamma"],
                                P["alpha"], P["ug"], P["ug_min"], P["normalize"])
    assert got.dtype == torch.float32
    close(got.cpu().numpy(), ref, RTOL[x["dtype"]], 1e-2)


@pytest.mark.parametrize("case", PW_CASES, ids=lambda c: c["name"])
def test_pairwise_dice(ml, case):
    x = make(6, **case["kw"])
    P = pw_params(case["p"])
    got = ml.forward_pw_dice_loss(x["z"], x["tgt"], P["smooth"], P["bg"], P["dscale"], P["ug"],
                                  P["ug_min"])
    ref = O.pairwise_dice(x["z64"], x["tgt_np"], P["smooth"], P["bg"], P["dscale"], P["ug"],
                          P["ug_min"])
    close(got.cpu().numpy(), ref, RTOL[x["dtype"]], 1e-2)


def test_pairwise_gt_rule_and_empty(ml):
    """GT slots come from targets.max()+1; all-negative targets give no columns."""
    x = make(7)
    t = x["tgt"].clone()
    t[t > 2] = 2
    assert ml.forward_pw_dice_loss(x["z"], t, 1.0, -1, 1.0, 1.0, 0.05).shape[-1] == 3
    assert ml.forward_pw_sigmoid_ce_loss(x["z"], t, 0, 1.0, 0.0, -1.0, 1.0, 0.05, True).shape[-1] == 2
    neg = torch.full_like(t, -1)
    assert ml.forward_pw_dice_loss(x["z"], neg, 1.0, -1, 1.0, 1.0, 0.05).shape[-1] == 0


DENSE_CASES = [
    dict(name="f32_s1", kw=dict(L=2), p={}),
    dict(name="bf16_s1", kw=dict(dtype="bfloat16", sigma=3.0), p={}),
    dict(name="f16_s2", kw=dict(dtype="float16", s=2, H=8, W=8), p={}),
    dict(name="f32_s4_focal", kw=dict(s=4, H=8, W=8, C=9), p=dict(gamma=2.0, alpha=0.25)),
    dict(name="f32_s17_u16_counts", kw=dict(s=17, H=3, W=5, C=4), p=dict(gamma=2.0, alpha=0.25)),
    dict(name="f32_focal_g15", kw=dict(C=3), p=dict(gamma=1.5, alpha=0.6)),
    dict(name="f32_odd_tail", kw=dict(H=7, W=5, C=4, B=3), p=dict(num_masks=2.5)),
    dict(name="f32_big_plane", kw=dict(H=96, W=96, C=3), p={}),
    dict(name="bf16_133", kw=dict(dtype="bfloat16", sigma=3.0, C=133, H=32, W=32), p={}),
]


def dense_params(p, L, B, C):
    d = dict(gamma=0.0, alpha=-1.0, num_masks=float(L * B * C), scale=1.7, smooth=0.5)
    d.update(p)
    return d


@pytest.mark.parametrize("case", DENSE_CASES, ids=lambda c: c["name"])
def test_sigmoid_ce_fwd_bwd(ml, case):
    x = make(8, **case["kw"])
    L, B, C = x["z"].shape[:3]
    P = dense_params(case["p"], L, B, C)
    got = ml.forward_sigmoid_ce_loss(x["z"], x["tgt"], P["num_masks"], P["scale"], P["gamma"],
                                     P["alpha"])
    ref = O.sigmoid_ce_loss(x["z64"], x["tgt_np"], P["num_masks"], P["scale"], P["gamma"],
                            P["alpha"])
    rt = RTOL[x["dtype"]]
    close(got.cpu().numpy(), ref, rt, 1e-2)
    g = torch.linspace(0.5, 1.5, L, device="cuda")
    grad = ml.backward_sigmoid_ce_loss(g, x["z"], x["tgt"], P["num_masks"], P["scale"], P["gamma"],
                                       P["alpha"])
    assert grad.dtype == x["z"].dtype and grad.shape == x["z"].shape
    rg = O.sigmoid_ce_backward(g.cpu().numpy(), x["z64"], x["tgt_np"], P["num_masks"], P["scale"],
                               P["gamma"], P["alpha"])
    close(grad.float().cpu().numpy(), rg, rt, 1e-2 * np.abs(rg).max(), STORE[x["dtype"]])


@pytest.mark.parametrize("case", DENSE_CASES, ids=lambda c: c["name"])
def test_dice_fwd_bwd(ml, case):
    x = make(9, **case["kw"])
    L, B, C = x["z"].shape[:3]
    P = dense_params(case["p"], L, B, C)
    loss, I, Pm, T = ml.forward_dice_loss(x["z"], x["tgt"], P["smooth"], P["num_masks"], P["scale"])
    rl, rI, rP, rT = O.dice_loss(x["z64"], x["tgt_np"], P["smooth"], P["num_masks"], P["scale"])
    rt = RTOL[x["dtype"]]
    close(loss.cpu().numpy(), rl, rt, 1e-2)
    close(I.cpu().numpy(), rI, rt, 1e-2)
    close(Pm.cpu().numpy(), rP, rt, 1e-2)
    close(T.cpu().numpy(), rT, 1e-6, 0.0)  # exact counts
    g = torch.linspace(0.5, 1.5, L, device="cuda")
    grad = ml.backward_dice_loss(g, x["z"], x["tgt"], I, Pm, T, P["smooth"], P["num_masks"],
                                 P["scale"])
    assert grad.dtype == x["z"].dtype
    canc = dice_grad_cancellation(g.cpu().numpy(), x["z64"], x["tgt_np"], I.cpu().numpy(),
                                  Pm.cpu().numpy(), T.cpu().numpy(), P["smooth"], P["num_masks"],
                                  P["scale"])
    # the backward's inputs are the forward's float32 I, P, T (as in the reference);
    # the oracle gets the same ones, since 2 n D - N2 (2 I + smooth) can cancel
    rg = O.dice_loss_backward(g.cpu().numpy(), x["z64"], x["tgt_np"], I.cpu().numpy(),
                              Pm.cpu().numpy(), T.cpu().numpy(), P["smooth"], P["num_masks"],
                              P["scale"])
    close(grad.float().cpu().numpy(), rg, rt, 1e-2 * np.abs(rg).max(), canc + STORE[x["dtype"]])


def test_dense_autograd_functions(ml):
    from mask_loss_amd.functions import DiceLossFunction, SigmoidCELossFunction
    x = make(10, L=2, C=6, dtype="bfloat16", sigma=3.0)
    z = x["z"].clone().requires_grad_(True)
    a = SigmoidCELossFunction.apply(z, x["tgt"], None, 1.2, 2.0, 0.25)
    b = DiceLossFunction.apply(z, x["tgt"], 1.0, None, 0.8)
    (a.sum() + 2.0 * b.sum()).backward()
    L, B, C = z.shape[:3]
    ones = np.ones(L)
    rg = (O.sigmoid_ce_backward(ones, x["z64"], x["tgt_np"], float(L * B * C), 1.2, 2.0, 0.25)
          + O.dice_loss_backward(2 * ones, x["z64"], x["tgt_np"],
                                 *O.dice_loss(x["z64"], x["tgt_np"], 1.0, float(L * B * C), 0.8)[1:],
                                 1.0, float(L * B * C), 0.8))
    close(z.grad.float().cpu().numpy(), rg, 2e-2, 1e-2 * np.abs(rg).max())


def test_dense_validation(ml):
    from mask_loss_amd.functions import PairwiseSigmoidCELossFunction, SigmoidCELossFunction
    x = make(11)
    with pytest.raises(ValueError, match="focal_alpha"):
        SigmoidCELossFunction.apply(x["z"], x["tgt"], None, 1.0, 0.0, 1.5)
    with pytest.raises(ValueError, match="uncertainty_gamma_min"):
        PairwiseSigmoidCELossFunction.apply(x["z"], x["tgt"], -1, 1.0, 0.0, None, 1.0, 2.0)
    bad = torch.zeros(2, 17, 16, dtype=torch.long, device="cuda")
    with pytest.raises(RuntimeError, match="integer multiple"):
        ml.forward_sigmoid_ce_loss(x["z"], bad, 1.0, 1.0, 0.0, -1.0)


def test_dense_deterministic(ml):
    x = make(12, C=40, H=64, W=64, dtype="bfloat16", sigma=3.0)
    a = ml.forward_dice_loss(x["z"], x["tgt"], 1.0, 7.0, 1.0)
    b = ml.forward_dice_loss(x["z"], x["tgt"], 1.0, 7.0, 1.0)
    for u, v in zip(a, b):
        assert torch.equal(u, v)
    assert torch.equal(ml.forward_sigmoid_ce_loss(x["z"], x["tgt"], 3.0, 1.0, 2.0, 0.25),
                       ml.forward_sigmoid_ce_loss(x["z"], x["tgt"], 3.0, 1.0, 2.0, 0.25))
