"""SigmoidCELossFunction -- reference functions/sigmoid/sigmoid_ce.py:22-70.

Count-based (focal) sigmoid cross entropy of dense class logits (L,B,C,h,w)
against a label map (B,H_t,W_t), one value per layer.  Same positional
signature, defaults and validation as the reference; the logits are consumed
in their own dtype (no float32 copy) and the gradient comes back in it."""
from __future__ import annotations

from torch.autograd import Function

import mask_loss_amd  # noqa: F401
import mask_loss


def _focal(focal_gamma, focal_alpha):
    gamma = 0.0 if focal_gamma is None else float(focal_gamma)
    if gamma < 0.0:
        raise ValueError("focal_gamma must be non-negative")
    if focal_alpha is None:
        alpha = -1.0
    else:
        alpha = float(focal_alpha)
        if not (0.0 <= alpha <= 1.0):
            raise ValueError("focal_alpha must be in [0, 1]")
    return gamma, alpha


class SigmoidCELossFunction(Function):
    @staticmethod
    def forward(ctx, logits, targets, num_masks, scale, focal_gamma, focal_alpha):
        L, B, C, h, w = logits.shape
        B_t, H_t, W_t = targets.shape
        assert B == B_t, "Batch size mismatch between logits and targets"
        if num_masks is None:
            num_masks = float(L * B * C)
        ctx.num_masks = num_masks
        ctx.scale = 1.0 if scale is None else float(scale)
        ctx.focal_gamma, ctx.focal_alpha = _focal(focal_gamma, focal_alpha)
        logits = logits.contiguous()
        targets = targets.contiguous()
        ctx.save_for_backward(logits, targets)
        return mask_loss.forward_sigmoid_ce_loss(logits, targets, num_masks, ctx.scale,
                                                 ctx.focal_gamma, ctx.focal_alpha)

    @staticmethod
    def backward(ctx, grad_output):
        logits, targets = ctx.saved_tensors
        grad = mask_loss.backward_sigmoid_ce_loss(grad_output.contiguous(), logits, targets,
                                                  ctx.num_masks, ctx.scale, ctx.focal_gamma,
                                                  ctx.focal_alpha)
        return grad, None, None, None, None, None
