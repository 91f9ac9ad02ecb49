"""PairwiseSigmoidCELossFunction -- reference
functions/sigmoid/pw_sigmoid_ce.py:17-73 (forward only).

Pairwise (focal) sigmoid cross entropy between every logit channel and every
GT slot of the label map, (L,B,C,GT_out); GT slots are 0..targets.max() as
in the reference.  Logits are consumed in their own dtype."""
from __future__ import annotations

from torch.autograd import Function

import mask_loss_amd  # noqa: F401
import mask_loss

from .._args import uncertainty
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
