"""PairwiseSigmoidLabelLossFunction -- reference
functions/label/pw_sigmoid_label_loss.py:12-52 (forward only)."""
from __future__ import annotations

from torch.autograd import Function

import mask_loss_amd  # noqa: F401
import mask_loss


class PairwiseSigmoidLabelLossFunction(Function):
    @staticmethod
    def forward(ctx, logits, targets, background_index=None, scale=1.0, focal_gamma=0.0,
                focal_alpha=None):
        gamma = 0.0 if focal_gamma is None else float(focal_gamma)
        if gamma < 0.0:
            raise ValueError("focal_gamma must be non-negative")
        if focal_alpha is None:
            alpha = -1.0
        else:
            alpha = float(focal_alpha)
            if not (0.0 <= alpha <= 1.0):
                raise ValueError("focal_alpha must be in [0, 1]")
        bg = -1 if background_index is None else int(background_index)
        return mask_loss.forward_pw_sigmoid_label_loss(
            logits.contiguous(), targets.contiguous(), bg,
            1.0 if scale is None else float(scale), gamma, alpha)

    @staticmethod
    def backward(ctx, grad_output):
        return None, None, None, None, None, None
