"""DiceLossFunction -- reference functions/dice/dice_loss.py:14-50.

Count-based dice loss of dense class logits (L,B,C,h,w) against a label map
(B,H_t,W_t), one value per layer; the per-(l,b,c) intersection, prediction
and target sums are kept for the backward, as in the reference.  Logits are
consumed in their own dtype and the gradient comes back in it."""
from __future__ import annotations

from torch.autograd import Function

import mask_loss_amd  # noqa: F401
import mask_loss


class DiceLossFunction(Function):
    @staticmethod
    def forward(ctx, logits, targets, smooth, num_masks, scale=1.0):
        L, B, C, h, w = logits.shape
        B_t, H_t, W_t = targets.shape
        assert B == B_t, "Batch size mismatch between logits and targets"
        if num_masks is None:
            num_masks = float(L * B * C)
        ctx.num_masks = num_masks
        ctx.scale = 1.0 if scale is None else float(scale)
        logits = logits.contiguous()
        targets = targets.contiguous().long()
        ctx.smooth = smooth
        output, int_sum, p_sum, t_sum = mask_loss.forward_dice_loss(logits, targets, smooth,
                                                                    num_masks, ctx.scale)
        ctx.save_for_backward(logits, targets, int_sum, p_sum, t_sum)
        return output

    @staticmethod
    def backward(ctx, grad_output):
        logits, targets, int_sum, p_sum, t_sum = ctx.saved_tensors
        grad = mask_loss.backward_dice_loss(grad_output.contiguous(), logits, targets, int_sum,
                                            p_sum, t_sum, ctx.smooth, ctx.num_masks, ctx.scale)
        return grad, None, None, None, None
