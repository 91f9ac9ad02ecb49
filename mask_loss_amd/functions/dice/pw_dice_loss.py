"""PairwiseDiceLossFunction -- reference functions/dice/pw_dice_loss.py:15-57
(forward only).

Pairwise dice cost between every logit channel and every GT slot of the label
map, (L,B,C,GT_out); GT slots are 0..targets.max() as in the reference.
Logits are consumed in their own dtype."""
from __future__ import annotations

from torch.autograd import Function

import mask_loss_amd  # noqa: F401
import mask_loss

from .._args import uncertainty


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
