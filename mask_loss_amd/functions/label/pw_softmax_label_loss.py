"""PairwiseSoftmaxLabelLossFunction -- reference
functions/label/pw_softmax_label_loss.py:13-50 (forward only)."""
from __future__ import annotations

from torch.autograd import Function

import mask_loss_amd  # noqa: F401
import mask_loss


class PairwiseSoftmaxLabelLossFunction(Function):
    @staticmethod
    def forward(ctx, logits, targets, background_index=None, scale=1.0):
        bg = -1 if background_index is None else int(background_index)
        return mask_loss.forward_pw_softmax_label_loss(
            logits.contiguous(), targets.contiguous(), bg, 1.0 if scale is None else float(scale))

    @staticmethod
    def backward(ctx, grad_output):
        return None, None, None, None


def pairwise_softmax_label_loss(logits, targets, background_index=None, scale=1.0):
    return PairwiseSoftmaxLabelLossFunction.apply(logits, targets, background_index, scale)
