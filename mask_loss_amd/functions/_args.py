"""Argument defaulting and validation shared by the autograd front-ends; the
rules restate functions/mask/matching.py:114-196 and
functions/mask/pw_mask.py:51-90 of the reference."""
from __future__ import annotations


def focal(mask_focal_gamma, mask_focal_alpha, cls_focal_gamma, cls_focal_alpha):
    mg = 0.0 if mask_focal_gamma is None else float(mask_focal_gamma)
    if mg < 0.0:
        raise ValueError("focal_gamma must be non-negative")
    if mask_focal_alpha is None:
        ma = -1.0
    else:
        ma = float(mask_focal_alpha)
        if not (0.0 <= ma <= 1.0):
            raise ValueError("focal_alpha must be in [0, 1]")
    if cls_focal_gamma is None:
        cg = mg
    else:
        cg = float(cls_focal_gamma)
        if cg < 0.0:
            raise ValueError("focal_gamma must be non-negative")
    if cls_focal_alpha is None:
        ca = ma
    else:
        ca = float(cls_focal_alpha)
        if not (0.0 <= ca <= 1.0):
            raise ValueError("focal_alpha must be in [0, 1]")
    return mg, ma, cg, ca


def uncertainty(uncertainty_gamma, uncertainty_gamma_min):
    ug = 1.0 if uncertainty_gamma is None else float(uncertainty_gamma)
    if ug < 0.0:
        raise ValueError("uncertainty_gamma must be non-negative")
    ugm = 0.05 if uncertainty_gamma_min is None else float(uncertainty_gamma_min)
    if not (0.0 <= ugm <= 1.0):
        raise ValueError("uncertainty_gamma_min must be in [0, 1]")
    return ug, ugm


def label_kind(label_loss):
    kind = (label_loss or "sigmoid").lower()
    if kind not in {"sigmoid", "softmax"}:
        raise ValueError("label_loss must be either 'sigmoid' or 'softmax'")
    return kind == "softmax"


STRATEGIES = {"global": 0, "round": 1, "greedy": 2, "pseudo_greedy": 3}
