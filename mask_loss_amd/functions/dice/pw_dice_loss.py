"""PairwiseDiceLossFunction -- reference functions/dice/pw_dice_loss.py:15-57
(forward only), and the point-sampled pairwise cost
pairwise_dice_loss_sampling_py (functions/dice/pw_dice_loss.py:174-268).

Pairwise dice cost between every logit channel and every GT slot of the label
map, (L,B,C,GT_out); GT slots are 0..targets.max() as in the reference.
Logits are consumed in their own dtype."""
from __future__ import annotations

import torch
from torch.autograd import Function

import mask_loss_amd  # noqa: F401
import mask_loss

from .._args import uncertainty
from ..sigmoid.pw_sigmoid_ce import _sampling_coords


class PairwiseDiceLossFunction(Function):
    @staticmethod
    def forward(ctx, logits, targets, smooth, background_index, scale, uncertainty_gamma=None,
                uncertainty_gamma_min=None):
        L, B, C, h, w = logits.shape
        B_t, H_t, W_t = targets.shape
        assert B == B_t, "Batch size mismatch between logits and targets"
        ug, ugm = uncertainty(uncertainty_gamma, uncertainty_gamma_min)
        return mask_loss.forward_pw_dice_loss(
            logits.contiguous(), targets.contiguous(),
            smooth if smooth is not None else 1.0,
            background_index if background_index is not None else -1,
            scale if scale is not None else 1.0, ug, ugm)

    @staticmethod
    def backward(ctx, grad_output):
        return (None,) * 7


def pairwise_dice_loss_sampling_py(
    logits, targets, smooth=1.0, background_index=None, scale=1.0, num_points=5000,
    align_corners=False, point_coords=None,
):
    """Pairwise dice cost on one shared set of points per image (reference
    functions/dice/pw_dice_loss.py:174-268), on the HIP path: (L, B, C, G) in
    the logits' dtype, +inf for classes absent from an image's label map.
    Points as in pairwise_sigmoid_cross_entropy_loss_sampling_py."""
    assert logits.dim() == 5, "logits must have shape (L, B, C, h, w)"
    L, B, C, h, w = logits.shape
    Bt, Ht, Wt = targets.shape
    assert B == Bt, "Batch size mismatch"
    coords = _sampling_coords(B, num_points, point_coords, logits.device, targets, background_index)
    out = mask_loss.forward_pw_dice_loss_sampling(
        logits.contiguous(), targets.to(device=logits.device, dtype=torch.long).contiguous(), coords,
        float(smooth if smooth is not None else 1.0),
        background_index if background_index is not None else -1,
        float(scale if scale is not None else 1.0), bool(align_corners))
    return out.to(logits.dtype)
