"""GPU parity at the full sizes of the benchmark configurations.

Every configuration of ``mask_loss_amd.synth.CONFIGS`` (the inputs bench.py
times) runs the fused step -- MaskMatchingFunction forward, then backward of
the sum of the layer means -- at its full size, and is checked:

* the assignment and pred_round of every image, bit for bit, against the C
  restatement of the reference solver on the GPU's own float32 cost matrix
  (reference src/cpu/matching.cpp:95-186, :476-571);
* the assignment of every image against the same solver on the float64
  oracle's costs of that image (all queries, all columns): equal, or not
  separated from the float64 optimum by more than rt * sum |matched costs|
  (the north star's index rule; at bfloat16 this covers the cost table's
  rounding of the four planes);
* the bce / dice / label costs of two full images (the ones with the most and
  the fewest non-empty GTs) against the float64 oracle (reference
  src/cuda/pw_mask.cu:52-308, src/cuda/pw_softmax_label_loss.cu:12-103);
* on every row of every image: +inf exactly where the GT is empty or its class
  invalid, bce >= 0, 0 <= dice < dice_scale, and each image's matched count
  equal to its number of valid columns (Q is larger in every configuration);
* the per-layer means against float64 sums of the GPU's costs at the
  assignment plus the oracle's unmatched-query class penalties, with the
  reference's denominators (src/cuda/mask_matching_forward.cu:21-279, :549-583);
* the mask-logit and class-logit gradients of every row of the two images
  against the float64 oracle with the batch's denominators
  (src/cuda/mask_matching_backward.cu); unmatched rows must be exactly zero.

cfg1 (the reference's CPU-runnable case) is compared with the oracle in full.
cfg2 also runs through the point-sampling front end, as bench.py does: dense
(1, 8, 100, 128, 128) logits sampled at 12,544 points per image.

Tolerances as the north star: float32 logits rel 1e-5, bfloat16 rel 2e-2,
|g - r| <= rtol (|r| + floor), floor 1e-2 for costs and losses and
1e-2 max|r| for gradients; indices bit-exact.
"""
import dataclasses

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import assign as OA  # noqa: E402
from oracle import mask_oracle as O  # noqa: E402
from oracle import points_oracle as PO  # noqa: E402
from assign_rule import check_f64_assignment_total  # noqa: E402

pytestmark = pytest.mark.gpu

RTOL = {"float32": 1e-5, "bfloat16": 2e-2}


@pytest.fixture(scope="module")
def ml():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mask_loss_amd
    return mask_loss_amd.mask_loss


def close(g, r, rtol, floor, what=""):
    g = np.asarray(g, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    assert g.shape == r.shape, (what, g.shape, r.shape)
    assert np.array_equal(np.isinf(g), np.isinf(r)), f"{what}: inf pattern differs"
    f = np.isfinite(r)
    err = np.abs(g[f] - r[f])
    bound = rtol * (np.abs(r[f]) + floor)
    bad = err > bound
    assert not bad.any(), f"{what}: max err {err.max():.3e}, worst ratio {(err / bound).max():.3f}"


def kw_args(cfg):
    k = cfg.kwargs
    return dict(smooth=k["smooth"], ss=k["sigmoid_scale"], ds=k["dice_scale"], cs=k["cls_scale"],
                bg=k["background_index"], ug=k["uncertainty_gamma"], ug_min=k["uncertainty_gamma_min"],
                void=cfg.C, softmax=k["label_loss"] == "softmax", force_cls=k["force_unmatched_class_to_background"],
                force_masks=k["force_unmatched_masks_to_empty"], num_masks=k["num_masks"],
                inf_thresh=k["inf_thresh"], K=k["K"])


def run_step(cfg, mask_logits, targets, cls_logits, cls_targets):
    """The benchmark's step: forward, then backward of the sum of the layer means."""
    from mask_loss_amd import synth
    from mask_loss_amd.functions import MaskMatchingFunction
    z = mask_logits.detach().clone().requires_grad_(True)
    zc = cls_logits.detach().clone().requires_grad_(True)
    args = synth.call_args(cfg, dict(mask_logits=z, mask_targets=targets, cls_logits=zc,
                                     cls_targets=cls_targets))
    p2g, pr, m, d, c = MaskMatchingFunction.apply(*args)
    torch.autograd.backward((m, d, c), [torch.ones(cfg.L, device="cuda")] * 3)
    torch.cuda.synchronize()
    return p2g, pr, torch.stack([m, d, c]), z.grad, zc.grad


def gpu_separate_costs(ml, cfg, z, t, zc, ct):
    a = kw_args(cfg)
    return ml.pairwise_mask_loss_forward(z, t, zc, ct, a["smooth"], a["ss"], a["ds"], a["cs"],
                                         a["bg"], a["ug"], a["ug_min"], 0.0, -1.0, 0.0, -1.0,
                                         a["softmax"], True)


def present_columns(tgt_np, GT_total, bg):
    """(B, GT_out) bool: the GT of output column k has a pixel."""
    B = tgt_np.shape[0]
    GT_out, bgn = O.column_layout(GT_total, bg)
    acts = np.array([O.out_to_actual(k, bgn) for k in range(GT_out)])
    pres = np.zeros((B, GT_out), dtype=bool)
    for b in range(B):
        cnt = np.bincount(tgt_np[b].reshape(-1).clip(-1, GT_total) + 1, minlength=GT_total + 2)[1:]
        pres[b] = cnt[acts] > 0
    return pres, acts


def oracle_image_costs(cfg, z, t, zc, ct):
    """The float64 oracle's separate costs (3, L, B, Q, G) of every image,
    one image per host thread (one BLAS thread each)."""
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits
    a = kw_args(cfg)
    B = t.shape[0]
    tgt_np = t.cpu().numpy()
    ct_np = ct.cpu().numpy()
    zc64 = zc.detach().double().cpu().numpy()

    def one(b):
        z64 = z.detach()[:, b:b + 1].double().cpu().numpy()
        return O.pairwise_mask_loss_forward(z64, tgt_np[b:b + 1], zc64[:, b:b + 1], ct_np[b:b + 1],
                                            a["smooth"], a["ss"], a["ds"], a["cs"], a["bg"], a["ug"],
                                            a["ug_min"], 0.0, -1.0, 0.0, -1.0, a["softmax"], True)

    with threadpool_limits(limits=1):
        with ThreadPoolExecutor(min(B, 16)) as ex:
            parts = list(ex.map(one, range(B)))
    return np.concatenate(parts, axis=2)


def check_step(ml, cfg, z, t, zc, ct, p2g, pr, means, gz, gzc, dtype, full_oracle=False,
               grad_map=None):
    """All checks of the module docstring on one step's results.  grad_map(b,
    rows, g_rows) -> (g_dense_gpu, g_dense_ref): optional mapping of sampled
    gradient rows to the input the step was differentiated against."""
    a = kw_args(cfg)
    rt = RTOL[dtype]
    L, B, Q = p2g.shape
    tgt_np = t.cpu().numpy()
    ct_np = ct.cpu().numpy()
    GT_total = ct_np.shape[1]
    C = zc.shape[-1]
    sep = gpu_separate_costs(ml, cfg, z.detach(), t, zc.detach(), ct).cpu().numpy()
    G = sep.shape[-1]
    p2g_np = p2g.cpu().numpy()
    # 1. assignment of every image, bit for bit, on the GPU's float32 costs
    total = ((torch.from_numpy(sep[0]) + torch.from_numpy(sep[1])) + torch.from_numpy(sep[2]))
    total = total.double().numpy().reshape(L * B, Q, G)
    rp2g, rpr = OA.assign_batch(total, a["inf_thresh"], a["K"], 0, nthreads=8)
    assert np.array_equal(p2g_np.reshape(L * B, Q), rp2g), "assignment differs from the reference solver"
    assert np.array_equal(pr.cpu().numpy().reshape(L * B, Q), rpr), "pred_round differs"
    # 1b. the north star's index rule on every image: the float64 oracle's
    # costs of all images, the reference solver on them, the GPU's indices
    # equal or within the cost tolerance of that optimum
    ref_all = oracle_image_costs(cfg, z, t, zc, ct)
    tot64 = ((ref_all[0] + ref_all[1]) + ref_all[2]).reshape(L * B, Q, G)
    _, ndiff = check_f64_assignment_total(tot64, p2g_np, rt, a["inf_thresh"], a["K"], 0,
                                          nthreads=8)
    print(f"{cfg.name}: {ndiff} of {L * B} slices differ from the float64 optimum (within tolerance)")
    # 2. properties on every row
    pres, acts = present_columns(tgt_np, GT_total, a["bg"])
    ycls = ct_np[:, acts]
    cls_ok = (ycls >= 0) & (ycls < C)
    for l in range(L):
        assert np.array_equal(np.isinf(sep[0, l]), np.broadcast_to(~pres[:, None, :], (B, Q, G)))
        assert np.array_equal(np.isinf(sep[1, l]), np.broadcast_to(~pres[:, None, :], (B, Q, G)))
        assert np.array_equal(np.isinf(sep[2, l]), np.broadcast_to(~cls_ok[:, None, :], (B, Q, G)))
    fin = np.isfinite(sep[0])
    assert (sep[0][fin] >= 0).all(), "negative bce"
    assert ((sep[1][fin] >= 0) & (sep[1][fin] < a["ds"])).all(), "dice outside [0, dice_scale)"
    nvalid = (pres & cls_ok).sum(1)
    matched = (p2g_np >= 0).sum(axis=2)
    assert np.array_equal(matched, np.broadcast_to(np.minimum(nvalid, Q), (L, B))), (matched, nvalid)
    # 3. means: float64 sums of the GPU's costs at the assignment, oracle penalties elsewhere
    zc64 = zc.detach().double().cpu().numpy()
    m = zc64.max(-1)
    lse = np.log(np.exp(zc64 - m[..., None]).sum(-1)) + m
    pen = (lse - zc64[..., a["void"]]) * a["cs"]  # softmax CE towards the no-object class
    md, cd = O.denominators(p2g_np, B, Q, a["num_masks"], a["force_masks"], a["force_cls"], True)
    exp = np.zeros((3, L))
    for l in range(L):
        for b in range(B):
            for q in range(Q):
                g = p2g_np[l, b, q]
                if g >= 0:
                    exp[:, l] += sep[:, l, b, q, g]
                else:
                    exp[2, l] += pen[l, b, q]
    exp[0] /= md
    exp[1] /= md
    exp[2] /= cd
    close(means.detach().cpu().numpy(), exp, rt, 1e-2, "layer means")
    # 4. two full images against the float64 oracle: costs, then gradients
    ngt = pres.sum(1)
    imgs = list(range(B)) if full_oracle else sorted({int(np.argmax(ngt)), int(np.argmin(ngt))})
    if len(imgs) == 1 and B > 1:
        imgs.append((imgs[0] + 1) % B)
    for b in imgs:
        z64 = z.detach()[:, b:b + 1].double().cpu().numpy()
        tb, cb = tgt_np[b:b + 1], ct_np[b:b + 1]
        ref = ref_all[:, :, b:b + 1]
        close(sep[0][:, b:b + 1], ref[0], rt, 1e-2, f"bce image {b}")
        close(sep[1][:, b:b + 1], ref[1], rt, 1e-2, f"dice image {b}")
        close(sep[2][:, b:b + 1], ref[2], 1e-5, 1e-2, f"label cost image {b}")
        pb = p2g_np[:, b:b + 1]
        rz, rzc = O.matching_backward(np.ones(L), np.ones(L), np.ones(L), z64, tb, zc64[:, b:b + 1],
                                      cb, pb, a["smooth"], a["ss"], a["ds"], a["cs"], a["bg"],
                                      a["ug"], a["ug_min"], a["num_masks"], a["force_cls"],
                                      a["force_masks"], void_class_index=a["void"],
                                      use_softmax=a["softmax"], denoms=(md, cd))
        close(gzc[:, b].cpu().numpy(), rzc[:, 0], 1e-5, 1e-2 * max(np.abs(rzc).max(), 1e-30),
              f"class-logit gradient image {b}")
        if grad_map is None:  # every row of the image
            got, want = gz[:, b].float().cpu().numpy(), rz[:, 0]
        else:  # sampled matched and unmatched rows, mapped to the differentiated input
            rng = np.random.default_rng(b)
            mq = np.flatnonzero(pb[0, 0] >= 0)
            uq = np.flatnonzero(pb[0, 0] < 0)
            qs = np.array(list(rng.choice(mq, size=min(6, mq.size), replace=False)) +
                          list(rng.choice(uq, size=min(3, uq.size), replace=False)), dtype=np.int64)
            got, want = grad_map(b, qs, rz[:, 0, qs])
        close(got, want, rt, 1e-2 * max(np.abs(want).max(), 1e-30), f"mask-logit gradient image {b}")
    return int(matched.sum())


DENSE = ["cfg1_cpu_ref", "cfg2_point_sampled", "cfg3_dense_headline", "cfg4_high_res",
         "cfg5_large_query"]


@pytest.mark.parametrize("name", DENSE)
def test_config_full_size(ml, name):
    from mask_loss_amd import synth
    cfg = synth.BY_NAME[name]
    x = synth.make_torch(cfg, "cuda", logits_on_device_rng=True)  # bench.py's inputs
    p2g, pr, means, gz, gzc = run_step(cfg, x["mask_logits"], x["mask_targets"], x["cls_logits"],
                                       x["cls_targets"])
    M = check_step(ml, cfg, x["mask_logits"], x["mask_targets"], x["cls_logits"], x["cls_targets"],
                   p2g, pr, means, gz, gzc, cfg.dtype, full_oracle=name == "cfg1_cpu_ref")
    print(f"{name}: matched {M}")


def test_config2_point_sampled_step(ml):
    """Configuration 2 as bench.py's Mask2Former-style step: dense
    (1, 8, 100, 128, 128) float32 logits, 512 x 512 label maps, 12,544 points
    per image; point_sample (autograd) into the fused step, gradient to the
    dense logits.  The samples and the labels under the points are checked
    against the points oracle, the rest as the dense configurations (costs on
    the sampled map), and the dense gradient rows against the oracle's
    adjoint of the sampling applied to the oracle's sampled-row gradients."""
    from mask_loss_amd import synth
    from mask_loss_amd.functions import MaskMatchingFunction, point_sample
    cfg = dataclasses.replace(synth.BY_NAME["cfg2_point_sampled"], H=128, W=128, scale=4)
    rng = np.random.Generator(np.random.PCG64(cfg.seed))
    labels, cls_t, _ = synth.make_targets(cfg, rng)
    t = torch.from_numpy(np.ascontiguousarray(labels)).cuda()
    g = torch.Generator(device="cuda")
    g.manual_seed(2)
    z = torch.randn(cfg.L, cfg.B, cfg.Q, cfg.H, cfg.W, device="cuda", generator=g) * cfg.sigma
    P = 12544
    coords = torch.rand(cfg.B, P, 2, device="cuda", generator=g)
    zc = torch.randn(cfg.L, cfg.B, cfg.Q, cfg.C + 1, device="cuda", generator=g)
    ct = torch.from_numpy(np.ascontiguousarray(cls_t)).cuda()
    lab = ml.point_labels(t, coords).view(cfg.B, 1, P)
    c_np = coords.cpu().numpy()
    assert np.array_equal(lab.view(cfg.B, P).cpu().numpy(), PO.point_labels(labels, c_np))
    zd = z.clone().requires_grad_(True)
    zcg = zc.clone().requires_grad_(True)
    zs = point_sample(zd.view(cfg.L * cfg.B, cfg.Q, cfg.H, cfg.W),
                      coords.repeat(cfg.L, 1, 1)).view(cfg.L, cfg.B, cfg.Q, 1, P)
    out = MaskMatchingFunction.apply(*synth.call_args(
        cfg, dict(mask_logits=zs, mask_targets=lab, cls_logits=zcg, cls_targets=ct)))
    torch.autograd.backward(out[2:], [torch.ones(cfg.L, device="cuda")] * 3)
    torch.cuda.synchronize()
    p2g, pr = out[0], out[1]
    means = torch.stack(list(out[2:]))
    zs_d = zs.detach()
    z_np = z.cpu().numpy()
    for b in (0, cfg.B - 1):  # samples of two images against the oracle
        ref = PO.point_sample(z_np[0, b:b + 1].astype(np.float64), c_np[b:b + 1])
        close(zs_d[0, b:b + 1, :, 0].cpu().numpy(), ref, 1e-5, np.abs(z_np[0, b]).max(), "samples")
    # the step on the sampled map: costs, assignment, losses, sampled-row gradients
    # (checked through the adjoint of the sampling, to the dense logits)
    gd = zd.grad.view(cfg.L, cfg.B, cfg.Q, cfg.H, cfg.W)

    def to_dense(b, qs, g_rows):
        # g_rows (L, n, 1, P): the oracle's gradient w.r.t. the sampled rows
        want = PO.point_sample_backward(g_rows.reshape(cfg.L, -1, P),
                                        np.repeat(c_np[b:b + 1], cfg.L, 0), cfg.H, cfg.W)
        return gd[:, b, qs].cpu().numpy(), want

    check_step(ml, cfg, zs_d, lab, zc, ct, p2g, pr, means, None, zcg.grad, "float32",
               grad_map=to_dense)
