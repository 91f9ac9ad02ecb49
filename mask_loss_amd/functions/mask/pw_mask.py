"""PairwiseMaskLossFunction -- reference functions/mask/pw_mask.py:21-115.

Forward returns the (3, L, B, Q, GT_out) [bce, dice, label] pairwise costs;
backward returns no gradients, as in the reference.  Logits are consumed in
their own dtype."""
from __future__ import annotations

from torch.autograd import Function

import mask_loss_amd  # noqa: F401
import mask_loss

from .._args import focal, label_kind, uncertainty


class PairwiseMaskLossFunction(Function):
    @staticmethod
    def forward(ctx, mask_logits, mask_targets, cls_logits, cls_targets, smooth, sigmoid_scale,
                dice_scale, cls_scale, background_index, uncertainty_gamma, uncertainty_gamma_min,
                normalize_uncertainty, mask_focal_gamma, mask_focal_alpha, cls_focal_gamma,
                cls_focal_alpha, label_loss: str = "sigmoid"):
        L, B, Q, h, w = mask_logits.shape
        assert B == mask_targets.shape[0], "Batch size mismatch between logits and targets"
        mg, ma, cg, ca = focal(mask_focal_gamma, mask_focal_alpha, cls_focal_gamma, cls_focal_alpha)
        ug, ugm = uncertainty(uncertainty_gamma, uncertainty_gamma_min)
        normalize = True if normalize_uncertainty is None else bool(normalize_uncertainty)
        use_softmax = label_kind(label_loss)
        return mask_loss.pairwise_mask_loss_forward(
            mask_logits.contiguous(), mask_targets.contiguous(), cls_logits.contiguous(),
            cls_targets.contiguous(),
            smooth if smooth is not None else 1.0,
            sigmoid_scale if sigmoid_scale is not None else 1.0,
            dice_scale if dice_scale is not None else 1.0,
            cls_scale if cls_scale is not None else 1.0,
            background_index if background_index is not None else -1,
            ug, ugm, mg, ma, cg, ca, use_softmax, normalize)

    @staticmethod
    def backward(ctx, grad_output):
        return (None,) * 17
