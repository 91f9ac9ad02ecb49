"""PairwiseSigmoidCELossFunction -- reference
functions/sigmoid/pw_sigmoid_ce.py:17-73 (forward only), and the point-sampled
pairwise cost pairwise_sigmoid_cross_entropy_loss_sampling_py
(functions/sigmoid/pw_sigmoid_ce.py:407-550).

Pairwise (focal) sigmoid cross entropy between every logit channel and every
GT slot of the label map, (L,B,C,GT_out); GT slots are 0..targets.max() as
in the reference.  Logits are consumed in their own dtype."""
from __future__ import annotations

import torch
from torch.autograd import Function

import mask_loss_amd  # noqa: F401
import mask_loss

from .._args import uncertainty
from ..utils import shared_point_coords
from .sigmoid_ce import _focal


class PairwiseSigmoidCELossFunction(Function):
    @staticmethod
    def forward(ctx, logits, targets, background_index, scale, focal_gamma, focal_alpha,
                uncertainty_gamma=None, uncertainty_gamma_min=None, normalize_uncertainty=True):
        L, B, C, h, w = logits.shape
        B_t, H_t, W_t = targets.shape
        assert B == B_t, "Batch size mismatch between logits and targets"
        fg, fa = _focal(focal_gamma, focal_alpha)
        ug, ugm = uncertainty(uncertainty_gamma, uncertainty_gamma_min)
        return mask_loss.forward_pw_sigmoid_ce_loss(
            logits.contiguous(), targets.contiguous(),
            background_index if background_index is not None else -1,
            scale if scale is not None else 1.0, fg, fa, ug, ugm,
            bool(normalize_uncertainty) if normalize_uncertainty is not None else True)

    @staticmethod
    def backward(ctx, grad_output):
        return (None,) * 9


def _sampling_coords(B, num_points, point_coords, device, targets=None, background_index=None):
    if point_coords is None:
        assert num_points > 0, "num_points must be > 0"
        return shared_point_coords(B, int(num_points), device, targets, background_index)
    assert point_coords.dim() == 3 and point_coords.shape[0] == B and point_coords.shape[2] == 2, \
        "point_coords must be (B, P, 2)"
    assert point_coords.shape[1] > 0, "num_points must be > 0"
    return point_coords.to(device=device, dtype=torch.float32).contiguous()


def pairwise_sigmoid_cross_entropy_loss_sampling_py(
    logits, targets, background_index=None, scale=1.0, num_points=5000, align_corners=False,
    focal_gamma=0.0, focal_alpha=None, point_coords=None,
):
    """Pairwise (focal) sigmoid CE on one shared set of points per image
    (reference functions/sigmoid/pw_sigmoid_ce.py:407-550), on the HIP path.

    logits (L, B, C, h, w), targets (B, H_t, W_t) -> (L, B, C, G) in the
    logits' dtype, G = targets.max() + 1 GT classes (minus the background),
    +inf for classes absent from an image's label map.  Predictions are
    sampled bilinearly at the points, labels by the floor mapping
    long(x * (W_t - 1)); the cost is the mean over the points.  The points
    are ``point_coords`` (B, P, 2) in [0, 1] if given, else ``num_points``
    drawn with ``torch.rand(1, P, 2)`` for the images the reference draws
    for (see shared_point_coords), in its order."""
    assert logits.dim() == 5, "logits must have shape (L, B, C, h, w)"
    L, B, C, h, w = logits.shape
    Bt, Ht, Wt = targets.shape
    assert B == Bt, "Batch size mismatch between logits and targets"
    fg, fa = _focal(focal_gamma, focal_alpha)
    coords = _sampling_coords(B, num_points, point_coords, logits.device, targets, background_index)
    out = mask_loss.forward_pw_sigmoid_ce_loss_sampling(
        logits.contiguous(), targets.to(device=logits.device, dtype=torch.long).contiguous(), coords,
        background_index if background_index is not None else -1,
        float(scale if scale is not None else 1.0), fg, fa, bool(align_corners))
    return out.to(logits.dtype)
