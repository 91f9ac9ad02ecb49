"""TEST INFRASTRUCTURE ONLY -- float64 CPU restatement of the reference's
fused pairwise mask-cost -> assignment -> matched-loss path.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  The product
path (``mask_loss_amd``) never imports it and has no CPU fallback.

Every function cites the reference file:line it restates (paths relative to
AndyBarcia/mask_loss).  Arithmetic is float64 throughout; the reference
computes in float32, so comparisons against it use the tolerances stated in
the tests.  The assignment solver is the C restatement in ``assign.c``
(loaded through ``oracle.assign``).

Pinning (which independent check fixes each function) is listed in the
module docstring of ``tests/test_oracle.py``; no function here is
"parity unpinned".
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

LOG2E = 1.4426950408889634
EPS = 1e-12


# ---------------------------------------------------------------------------
# target preparation
# ---------------------------------------------------------------------------
def label_counts(targets: np.ndarray, H: int, W: int, GT_total: int) -> np.ndarray:
    """Per-cell label counts, reference src/cuda/utils.cuh:6-36.

    targets: (B, H_t, W_t) integer labels.  Returns (B, GT_total, H*W) int64
    with n[b,g,cell] = number of high-res pixels of the s x s block of `cell`
    whose label is g.  Labels outside [0, GT_total) are ignored (utils.cuh:29).
    """
    B, Ht, Wt = targets.shape
    s = Ht // H
    assert Ht == s * H and Wt == s * W
    t = np.asarray(targets, dtype=np.int64).reshape(B, H, s, W, s)
    t = t.transpose(0, 1, 3, 2, 4).reshape(B, H * W, s * s)
    out = np.zeros((B, GT_total, H * W), dtype=np.int64)
    for g in range(GT_total):
        out[:, g, :] = (t == g).sum(axis=2)
    return out


def out_to_actual(k: int, bg: int) -> int:
    """Compacted column -> GT slot, reference src/cuda/utils.cuh:38-40."""
    return k + (1 if k >= bg else 0)


def column_layout(GT_total: int, background_index: int):
    """(GT_out, normalised bg), reference src/cuda/pw_mask.cu:394-399."""
    skip = 0 <= background_index < GT_total
    bg = background_index if background_index >= 0 else GT_total
    return GT_total - (1 if skip else 0), bg


# ---------------------------------------------------------------------------
# per-element quantities
# ---------------------------------------------------------------------------
@dataclass
class Elem:
    p: np.ndarray
    cp: np.ndarray  # softplus(-z) = -log p
    cn: np.ndarray  # softplus(z)  = -log(1-p)
    w: np.ndarray   # clamped entropy weight
    mp: np.ndarray  # (1-p)^gamma or 1
    mn: np.ndarray  # p^gamma or 1


def elementwise(z, gamma=0.0, ug=1.0, ug_min=0.05) -> Elem:
    """Per-logit terms, reference src/cuda/pw_mask.cu:124-142 and :250-267."""
    z = np.asarray(z, dtype=np.float64)
    a = np.abs(z)
    l1 = np.log1p(np.exp(-a))
    cn = l1 + np.maximum(z, 0.0)
    cp = l1 + np.maximum(-z, 0.0)
    p = 1.0 / (1.0 + np.exp(-z))
    pc = np.clip(p, EPS, 1.0 - EPS)
    with np.errstate(divide="ignore", invalid="ignore"):
        ent = -(pc * np.log(pc) + (1.0 - pc) * np.log(1.0 - pc)) * LOG2E
    if ug != 0.0:
        w = np.power(ent, ug)
    else:
        w = np.ones_like(z)
    w = np.minimum(1.0, np.maximum(w, ug_min))
    if gamma > 0.0:
        mp = np.power(1.0 - p, gamma)
        mn = np.power(p, gamma)
    else:
        mp = np.ones_like(z)
        mn = np.ones_like(z)
    return Elem(p=p, cp=cp, cn=cn, w=w, mp=mp, mn=mn)


def _alphas(alpha):
    """Focal alpha convention, reference src/cuda/pw_mask.cu:94-95."""
    return (alpha, 1.0 - alpha) if alpha >= 0.0 else (1.0, 1.0)


# ---------------------------------------------------------------------------
# pairwise costs
# ---------------------------------------------------------------------------
def pairwise_mask_costs(mask_logits, mask_targets, GT_total, background_index,
                        smooth=1.0, sigmoid_scale=1.0, dice_scale=1.0,
                        ug=1.0, ug_min=0.05, mask_gamma=0.0, mask_alpha=-1.0,
                        normalize=True):
    """BCE and dice pairwise costs, reference src/cuda/pw_mask.cu:52-308
    (kernel) and :314-445 (host: GT_total, GT_out, background column).

    Returns (bce, dice) each (L, B, Q, GT_out) float64, +inf for GT slots with
    zero area (pw_mask.cu:209-217).
    """
    z = np.asarray(mask_logits, dtype=np.float64)
    L, B, Q, H, W = z.shape
    _, Ht, Wt = mask_targets.shape
    s = Ht // H
    N2 = float(s * s)
    GT_out, bg = column_layout(GT_total, background_index)
    counts = label_counts(mask_targets, H, W, GT_total).astype(np.float64)  # (B,G,HW)
    area = counts.sum(axis=2)  # (B, G)
    ap, an = _alphas(mask_alpha)
    # every output column k at once: n[b, j, k] = count of GT slot a(k) at cell j
    acts = np.array([out_to_actual(k, bg) for k in range(GT_out)], dtype=np.int64)
    nT = np.ascontiguousarray(np.swapaxes(counts[:, acts, :], 1, 2))  # (B, HW, GT_out)
    empty = area[:, acts] == 0                         # pw_mask.cu:209-217
    bce = np.empty((L, B, Q, GT_out))
    dice = np.empty((L, B, Q, GT_out))
    zr = z.reshape(L, B, Q, H * W)
    # query rows in chunks of about 2^22 logits (bounded temporaries)
    rows = max(1, (1 << 22) // max(1, H * W))
    for l in range(L):
        for b in range(B):
            for q0 in range(0, Q, rows):
                e = elementwise(zr[l, b, q0:q0 + rows], mask_gamma, ug, ug_min)
                coeff_neg = an * e.mn * e.cn
                coeff_pos = ap * e.mp * e.cp
                base = (N2 * e.w * coeff_neg).sum(-1)          # pw_mask.cu:139
                p_total = (N2 * e.w * e.p).sum(-1)             # pw_mask.cu:140
                wsum = (N2 * e.w).sum(-1)                      # pw_mask.cu:141
                if not normalize:
                    wsum = np.full_like(wsum, float(Ht * Wt))  # pw_mask.cu:200-202
                wsum = np.maximum(wsum, EPS)                   # pw_mask.cu:203
                d = (e.w * (coeff_pos - coeff_neg)) @ nT[b]    # pw_mask.cu:268-271
                inter = (e.w * e.p) @ nT[b]
                tsum = e.w @ nT[b]
                bk = (base[:, None] + d) / wsum[:, None] * sigmoid_scale   # pw_mask.cu:300
                dk = (1.0 - (2.0 * inter + smooth) / (p_total[:, None] + tsum + smooth)) * dice_scale
                bce[l, b, q0:q0 + rows] = np.where(empty[b][None, :], np.inf, bk)
                dice[l, b, q0:q0 + rows] = np.where(empty[b][None, :], np.inf, dk)
    return bce, dice


def pairwise_sigmoid_label_cost(cls_logits, cls_targets, background_index,
                                scale=1.0, gamma=0.0, alpha=-1.0):
    """Reference src/cuda/pw_sigmoid_label_loss.cu:16-106 (+host :133-139)."""
    z = np.asarray(cls_logits, dtype=np.float64)
    L, B, Q, C = z.shape
    GT_total = cls_targets.shape[1]
    GT_out, bg = column_layout(GT_total, background_index)
    ap, an = _alphas(alpha)
    e = elementwise(z, gamma, 0.0, 0.0)
    neg = an * e.mn * e.cn
    pos = ap * e.mp * e.cp
    base = neg.sum(-1)
    out = np.empty((L, B, Q, GT_out))
    for k in range(GT_out):
        a = out_to_actual(k, bg)
        for b in range(B):
            y = int(cls_targets[b, a])
            if y < 0 or y >= C:
                out[:, b, :, k] = np.inf
            else:
                out[:, b, :, k] = (base[:, b, :] + pos[:, b, :, y] - neg[:, b, :, y]) / C * scale
    return out


def pairwise_softmax_label_cost(cls_logits, cls_targets, background_index, scale=1.0):
    """Reference src/cuda/pw_softmax_label_loss.cu:12-103."""
    z = np.asarray(cls_logits, dtype=np.float64)
    L, B, Q, C = z.shape
    GT_total = cls_targets.shape[1]
    GT_out, bg = column_layout(GT_total, background_index)
    m = z.max(-1)
    lse = np.log(np.maximum(np.exp(z - m[..., None]).sum(-1), 1e-20)) + m
    out = np.empty((L, B, Q, GT_out))
    for k in range(GT_out):
        a = out_to_actual(k, bg)
        for b in range(B):
            y = int(cls_targets[b, a])
            if y < 0 or y >= C:
                out[:, b, :, k] = np.inf
            else:
                out[:, b, :, k] = (lse[:, b, :] - z[:, b, :, y]) * scale
    return out


def pairwise_mask_loss_forward(mask_logits, mask_targets, cls_logits, cls_targets,
                               smooth=1.0, sigmoid_scale=1.0, dice_scale=1.0,
                               cls_scale=1.0, background_index=-1, ug=1.0,
                               ug_min=0.05, mask_gamma=0.0, mask_alpha=-1.0,
                               cls_gamma=0.0, cls_alpha=-1.0, use_softmax=False,
                               normalize=True):
    """(3, L, B, Q, GT_out) = [bce, dice, cls], reference src/cuda/pw_mask.cu:314-501."""
    GT_total = cls_targets.shape[1]
    bce, dice = pairwise_mask_costs(mask_logits, mask_targets, GT_total, background_index,
                                    smooth, sigmoid_scale, dice_scale, ug, ug_min,
                                    mask_gamma, mask_alpha, normalize)
    if use_softmax:
        cls = pairwise_softmax_label_cost(cls_logits, cls_targets, background_index, cls_scale)
    else:
        cls = pairwise_sigmoid_label_cost(cls_logits, cls_targets, background_index,
                                          cls_scale, cls_gamma, cls_alpha)
    return np.stack([bce, dice, cls])


# ---------------------------------------------------------------------------
# standalone pairwise costs (GT slots from the label map itself)
# ---------------------------------------------------------------------------
def gt_total_from_targets(targets) -> int:
    """GT_total = targets.max() + 1, reference src/cuda/pw_sigmoid_ce.cu:222-224
    and src/cuda/pw_dice_loss.cu:132-134 (not the cls_targets width)."""
    t = np.asarray(targets)
    return max(int(t.max()) + 1, 0) if t.size else 0


def pairwise_sigmoid_ce(logits, targets, background_index=-1, scale=1.0, gamma=0.0,
                        alpha=-1.0, ug=1.0, ug_min=0.05, normalize=True):
    """(L, B, C, GT_out), reference src/cuda/pw_sigmoid_ce.cu:12-197 (kernel: the
    BCE half of pw_mask.cu's) and :199-316 (host)."""
    bce, _ = pairwise_mask_costs(logits, targets, gt_total_from_targets(targets),
                                 background_index, 1.0, scale, 1.0, ug, ug_min, gamma, alpha,
                                 normalize)
    return bce


def pairwise_dice(logits, targets, smooth=1.0, background_index=-1, scale=1.0, ug=1.0,
                  ug_min=0.05):
    """(L, B, C, GT_out), reference src/cuda/pw_dice_loss.cu:12-108 (kernel:
    I = sum w p n, P = sum N2 w p, T = sum w n) and :111-221 (host)."""
    _, dice = pairwise_mask_costs(logits, targets, gt_total_from_targets(targets),
                                  background_index, smooth, 1.0, scale, ug, ug_min)
    return dice


# ---------------------------------------------------------------------------
# non-pairwise (per-class) losses over dense class logits
# ---------------------------------------------------------------------------
def sigmoid_ce_loss(logits, targets, num_masks, scale=1.0, gamma=0.0, alpha=-1.0):
    """(L,), reference src/cuda/sigmoid_ce.cu:13-114 (kernel) and :207-268 (host):
    sum over (b, c, cell) of ap mp cp n + an mn cn (N2 - n), n = count of class c
    in the cell's s x s block, times scale / (num_masks Ht Wt)."""
    z = np.asarray(logits, dtype=np.float64)
    L, B, C, H, W = z.shape
    _, Ht, Wt = targets.shape
    N2 = float((Ht // H) ** 2)
    n = label_counts(targets, H, W, C).astype(np.float64)   # (B, C, HW)
    e = elementwise(z.reshape(L, B, C, H * W), gamma, 0.0, 0.0)
    ap, an = _alphas(alpha)
    loss = ap * e.mp * e.cp * n + an * e.mn * e.cn * (N2 - n)
    return loss.sum(axis=(1, 2, 3)) * scale / (num_masks * Ht * Wt)


def sigmoid_ce_backward(grad_out, logits, targets, num_masks, scale=1.0, gamma=0.0,
                        alpha=-1.0):
    """(L, B, C, H, W), reference src/cuda/sigmoid_ce.cu:116-205 and :270-332:
    -ap n mp (gamma p cp + 1-p) + an (N2-n) mn (gamma (1-p) cn + p), times
    grad_out[l] scale / (num_masks Ht Wt)."""
    z = np.asarray(logits, dtype=np.float64)
    L, B, C, H, W = z.shape
    _, Ht, Wt = targets.shape
    N2 = float((Ht // H) ** 2)
    n = label_counts(targets, H, W, C).astype(np.float64).reshape(1, B, C, H, W)
    e = elementwise(z, gamma, 0.0, 0.0)
    ap, an = _alphas(alpha)
    g = (-ap * n * e.mp * (gamma * e.p * e.cp + (1.0 - e.p))
         + an * (N2 - n) * e.mn * (gamma * (1.0 - e.p) * e.cn + e.p))
    coef = np.asarray(grad_out, dtype=np.float64).reshape(L, 1, 1, 1, 1) * scale / (num_masks * Ht * Wt)
    return g * coef


def dice_loss(logits, targets, smooth, num_masks, scale=1.0):
    """(loss (L,), I, P, T (L, B, C)), reference src/cuda/dice_loss.cu:13-82 and
    :159-222: I = sum p n, P = sum N2 p, T = sum n; loss = scale / num_masks *
    sum_{b,c} 1 - (2I + smooth) / (P + T + smooth)."""
    z = np.asarray(logits, dtype=np.float64)
    L, B, C, H, W = z.shape
    _, Ht, Wt = targets.shape
    N2 = float((Ht // H) ** 2)
    n = label_counts(targets, H, W, C).astype(np.float64)   # (B, C, HW)
    p = 1.0 / (1.0 + np.exp(-z.reshape(L, B, C, H * W)))
    I = (p * n).sum(-1)
    P = N2 * p.sum(-1)
    T = np.broadcast_to(n.sum(-1), I.shape).copy()
    dice = (2.0 * I + smooth) / (P + T + smooth)
    loss = (1.0 - dice).reshape(L, -1).sum(1) / num_masks * scale
    return loss, I, P, T


def dice_loss_backward(grad_out, logits, targets, I, P, T, smooth, num_masks, scale=1.0):
    """(L, B, C, H, W), reference src/cuda/dice_loss.cu:84-157 and :224-289:
    -grad_out[l] scale / num_masks * (2 n D - N2 (2I + smooth)) / D^2 * p (1-p),
    D = P + T + smooth, with the forward's I, P, T."""
    z = np.asarray(logits, dtype=np.float64)
    L, B, C, H, W = z.shape
    _, Ht, Wt = targets.shape
    N2 = float((Ht // H) ** 2)
    n = label_counts(targets, H, W, C).astype(np.float64).reshape(1, B, C, H, W)
    p = 1.0 / (1.0 + np.exp(-z))
    I = np.asarray(I, dtype=np.float64)[..., None, None]
    D = (np.asarray(P, dtype=np.float64) + np.asarray(T, dtype=np.float64) + smooth)[..., None, None]
    g = (2.0 * n * D - N2 * (2.0 * I + smooth)) / (D * D) * p * (1.0 - p)
    coef = -np.asarray(grad_out, dtype=np.float64).reshape(L, 1, 1, 1, 1) / num_masks * scale
    return g * coef


# ---------------------------------------------------------------------------
# matched-loss forward
# ---------------------------------------------------------------------------
def denominators(pred_to_gt, B, Q, num_masks, force_masks, force_cls, has_void):
    """Per-layer denominators, reference src/cuda/mask_matching_forward.cu:549-574
    (identical rules in mask_matching_backward.cu:483-508)."""
    matched = (np.asarray(pred_to_gt) >= 0).sum(axis=(1, 2)).astype(np.float64)
    total = np.full_like(matched, float(B * Q))
    if force_masks:
        md = total.copy()
    elif num_masks > 0:
        md = np.full_like(matched, float(num_masks))
    else:
        md = matched.copy()
    if force_cls or has_void:
        cd = total.copy()
    elif num_masks > 0:
        cd = np.full_like(matched, float(num_masks))
    else:
        cd = matched.copy()
    return np.maximum(md, 1.0), np.maximum(cd, 1.0)


def matching_forward_losses(separate_costs, pred_to_gt, mask_logits, cls_logits,
                            mask_targets_shape, smooth=1.0, sigmoid_scale=1.0,
                            dice_scale=1.0, cls_scale=1.0, mask_gamma=0.0,
                            mask_alpha=-1.0, cls_gamma=0.0, cls_alpha=-1.0,
                            num_masks=-1.0, force_masks=False, force_cls=False,
                            void_class_index=-1, use_softmax=False):
    """Per-layer (mask, dice, cls) means, reference
    src/cuda/mask_matching_forward.cu:21-279 (kernel) and :283-586 (host)."""
    z = np.asarray(mask_logits, dtype=np.float64)
    L, B, Q, H, W = z.shape
    zc = np.asarray(cls_logits, dtype=np.float64)
    C = zc.shape[-1]
    Ht, Wt = mask_targets_shape[1], mask_targets_shape[2]
    area_scale = float((Ht // H) * (Wt // W)) if force_masks else 1.0
    void = void_class_index if 0 <= void_class_index < C else -1
    has_void = void >= 0
    if use_softmax and force_cls and not has_void:
        raise ValueError("void_class_index must be provided when using softmax label loss "
                         "and forcing unmatched class logits")
    softmax_bg = use_softmax and force_cls and has_void
    ap_m, an_m = _alphas(mask_alpha)
    use_cls_focal = not use_softmax
    ap_c, an_c = _alphas(cls_alpha) if use_cls_focal else (1.0, 1.0)
    g_c = cls_gamma if use_cls_focal else 0.0
    sums = np.zeros((3, L))
    p2g = np.asarray(pred_to_gt)
    for l in range(L):
        for b in range(B):
            for q in range(Q):
                g = int(p2g[l, b, q])
                if g >= 0:
                    sums[:, l] += separate_costs[:, l, b, q, g]
                    continue
                if force_masks:
                    e = elementwise(z[l, b, q].reshape(-1), mask_gamma, 0.0, 0.0)
                    bce_mean = (an_m * e.mn * e.cn).sum() / float(H * W)
                    psum = e.p.sum() * area_scale
                    sums[0, l] += sigmoid_scale * bce_mean
                    sums[1, l] += dice_scale * (psum / (psum + smooth))
                if force_cls or has_void:
                    zz = zc[l, b, q]
                    if softmax_bg:
                        m = zz.max()
                        lse = math.log(max(np.exp(zz - m).sum(), 1e-20)) + m
                        sums[2, l] += (lse - zz[void]) * cls_scale
                    else:
                        e = elementwise(zz, g_c, 0.0, 0.0)
                        neg = an_c * e.mn * e.cn
                        if force_cls:
                            loss = neg.sum() / C if C > 0 else 0.0
                            if has_void and C > 0:
                                vpos = ap_c * e.mp[void] * e.cp[void]
                                loss += (vpos - neg[void]) / C
                        else:
                            loss = ap_c * e.mp[void] * e.cp[void]
                        sums[2, l] += loss * cls_scale
    md, cd = denominators(p2g, B, Q, num_masks, force_masks, force_cls, has_void)
    return sums[0] / md, sums[1] / md, sums[2] / cd


# ---------------------------------------------------------------------------
# matched-loss backward
# ---------------------------------------------------------------------------
def matching_backward(g_mask, g_dice, g_cls, mask_logits, mask_targets, cls_logits,
                      cls_targets, pred_to_gt, smooth=1.0, sigmoid_scale=1.0,
                      dice_scale=1.0, cls_scale=1.0, background_index=-1, ug=1.0,
                      ug_min=0.05, num_masks=-1.0, force_cls=False, force_masks=False,
                      mask_gamma=0.0, mask_alpha=-1.0, cls_gamma=0.0, cls_alpha=-1.0,
                      void_class_index=-1, use_softmax=False, normalize=True,
                      denoms=None, rows=None):
    """(grad_mask_logits, grad_cls_logits), reference
    src/cuda/mask_matching_backward.cu:21-216 (mask kernel), :218-376 (class
    kernel) and :378-621 (host: denominators, counts, coefficients).
    Uncertainty weights and their normaliser are constants (detached).

    denoms: (mask, cls) per-layer denominators to use instead of those of
    `pred_to_gt` (a slice of a larger batch); rows: only these (l, b, q) rows
    are computed, the others stay zero."""
    z = np.asarray(mask_logits, dtype=np.float64)
    L, B, Q, H, W = z.shape
    zc = np.asarray(cls_logits, dtype=np.float64)
    C = zc.shape[-1]
    GT_total = cls_targets.shape[1]
    Ht, Wt = mask_targets.shape[1], mask_targets.shape[2]
    s = Ht // H
    area = float(s * s)
    bg = background_index if background_index >= 0 else GT_total
    void = void_class_index if 0 <= void_class_index < C else -1
    has_void = void >= 0
    if use_softmax and force_cls and not has_void:
        raise ValueError("void_class_index must be provided when using softmax label loss "
                         "and forcing unmatched class logits")
    need_cls = force_cls or has_void
    p2g = np.asarray(pred_to_gt)
    md, cd = denominators(p2g, B, Q, num_masks, force_masks, force_cls, has_void)
    if denoms is not None:
        md, cd = (np.asarray(v, dtype=np.float64).reshape(L) for v in denoms)
    inv_md = 1.0 / md
    cls_coeff = cls_scale / cd
    counts = label_counts(mask_targets, H, W, GT_total).astype(np.float64)
    ap, an = _alphas(mask_alpha)
    gm = np.zeros_like(z)
    gc = np.zeros_like(zc)
    g_mask = np.asarray(g_mask, dtype=np.float64)
    g_dice = np.asarray(g_dice, dtype=np.float64)
    g_cls = np.asarray(g_cls, dtype=np.float64)
    todo = rows if rows is not None else [(l, b, q) for l in range(L) for b in range(B)
                                          for q in range(Q)]
    for l, b, q in todo:
        out = int(p2g[l, b, q])
        act = out + (1 if out >= bg else 0)
        matched = out >= 0 and act < GT_total
        # ---- mask logits (mask_matching_backward.cu:47-215)
        if matched or force_masks:
            mc = g_mask[l] * inv_md[l]
            dc = g_dice[l] * inv_md[l]
            if not (mc == 0.0 and dc == 0.0):
                zz = z[l, b, q].reshape(-1)
                e = elementwise(zz, mask_gamma, ug, ug_min)
                t = counts[b, act] if matched else np.zeros_like(zz)
                P = (e.w * e.p * area).sum()
                T = (e.w * t).sum()
                I = (e.w * e.p * t).sum()
                S = (e.w * area).sum() if normalize else area * H * W
                S = max(S, EPS)
                D = P + T + smooth
                num = 2.0 * I + smooth
                D2 = max(D * D, 1e-20)
                negc = np.maximum(area - t, 0.0)
                gpos = -e.w * ap * t * e.mp * (mask_gamma * e.p * e.cp + (1.0 - e.p))
                gneg = e.w * an * negc * e.mn * (mask_gamma * (1.0 - e.p) * e.cn + e.p)
                gs = (gpos + gneg) * sigmoid_scale / S
                pp = e.p * (1.0 - e.p)
                gd = (num * e.w * pp * area - 2.0 * D * e.w * pp * t) / D2 * dice_scale
                gm[l, b, q] = (mc * gs + dc * gd).reshape(H, W)
        # ---- class logits (mask_matching_backward.cu:239-375)
        if not (matched or need_cls):
            continue
        base = g_cls[l] * cls_coeff[l]
        if base == 0.0:
            continue
        y = -1
        if matched:
            y = int(cls_targets[b, act])
            if y < 0 or y >= C:
                continue
        zz = zc[l, b, q]
        if use_softmax:
            if matched or (force_cls and has_void):
                tgt = y if matched else void
                m = zz.max()
                ex = np.exp(zz - m)
                sm = ex / ex.sum()
                gr = sm.copy()
                gr[tgt] -= 1.0
                gc[l, b, q] = base * gr
            elif has_void:
                gr = np.zeros(C)
                gr[void] = base * (1.0 / (1.0 + math.exp(-zz[void])) - 1.0)
                gc[l, b, q] = gr
            continue
        cap, can = _alphas(cls_alpha)
        e = elementwise(zz, cls_gamma, 0.0, 0.0)
        posg = -cap * e.mp * (cls_gamma * e.p * e.cp + (1.0 - e.p))
        negg = can * e.mn * (cls_gamma * (1.0 - e.p) * e.cn + e.p)
        if matched:
            gr = negg.copy()
            gr[y] = posg[y]
            gc[l, b, q] = base / C * gr
        elif force_cls:
            gr = negg.copy()
            if has_void:
                gr[void] = posg[void]
            gc[l, b, q] = base / C * gr
        elif has_void:
            gr = np.zeros(C)
            gr[void] = base * posg[void]
            gc[l, b, q] = gr
    return gm, gc


# ---------------------------------------------------------------------------
# full forward (costs -> assignment -> losses)
# ---------------------------------------------------------------------------
def mask_matching(mask_logits, mask_targets, cls_logits, cls_targets, smooth=1.0,
                  sigmoid_scale=1.0, dice_scale=1.0, cls_scale=1.0, background_index=-1,
                  ug=1.0, ug_min=0.05, inf_thresh=1e30, num_masks=-1.0,
                  force_cls=False, force_masks=False, topk=1, strategy=0,
                  mask_gamma=0.0, mask_alpha=-1.0, cls_gamma=0.0, cls_alpha=-1.0,
                  void_class_index=-1, use_softmax=False, normalize=True,
                  total_cost=None):
    """Reference src/cpu/matching.cpp:592-752.  Returns
    (pred_to_gt, pred_round, mask_mean, dice_mean, cls_mean, separate_costs).

    ``total_cost`` (L,B,Q,GT_out), if given, replaces the summed cost matrix fed
    to the assignment (used to run the solver on a cost matrix produced
    elsewhere, bit for bit)."""
    from . import assign as _assign
    sep = pairwise_mask_loss_forward(mask_logits, mask_targets, cls_logits, cls_targets,
                                     smooth, sigmoid_scale, dice_scale, cls_scale,
                                     background_index, ug, ug_min, mask_gamma, mask_alpha,
                                     cls_gamma, cls_alpha, use_softmax, normalize)
    cost = sep.sum(0) if total_cost is None else np.asarray(total_cost, dtype=np.float64)
    L, B, Q, GT_out = cost.shape
    p2g, pr = _assign.assign_batch(cost.reshape(L * B, Q, GT_out), inf_thresh, topk, strategy)
    p2g = p2g.reshape(L, B, Q)
    pr = pr.reshape(L, B, Q)
    m, d, c = matching_forward_losses(sep, p2g, mask_logits, cls_logits, mask_targets.shape,
                                      smooth, sigmoid_scale, dice_scale, cls_scale, mask_gamma,
                                      mask_alpha, cls_gamma, cls_alpha, num_masks, force_masks,
                                      force_cls, void_class_index, use_softmax)
    return p2g, pr, m, d, c, sep
