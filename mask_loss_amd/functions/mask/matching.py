"""MaskMatchingFunction -- reference functions/mask/matching.py:21-334.

Same positional signature, defaults and validation as the reference.  The
differences:

* mask logits are consumed in their own dtype (float32, bfloat16 or float16):
  no float32 copy of the logits is made (reference: ``.contiguous().float()``,
  matching.py:109-112); gradients come back in the logits' dtype, which is
  what autograd produces from the reference's float32 gradients;
* the forward keeps per-query statistics (uncertainty normaliser, mass,
  intersection, target mass), the matched rows and the compact label map, so
  the backward reads every matched logit once instead of twice (reference
  backward: mask_matching_backward.cu:110-215) and skips target preparation;
* when the mask logits need a gradient (and unmatched masks are not forced to
  empty, so unmatched rows have zero gradient), the forward allocates the
  gradient tensor and zero-fills it with extra workgroups of its own launches
  while the assignment runs; the first backward then writes only the matched
  rows into it;
* the autograd node is a C++ one (the extension's MatchingNode): the Python
  class applies the reference's defaults and validation only.
"""
from __future__ import annotations

from torch.autograd import Function

import mask_loss_amd  # noqa: F401  (registers the `mask_loss` module)
import mask_loss

from .._args import STRATEGIES, focal, label_kind, uncertainty


class MaskMatchingFunction(Function):
    """The reference's autograd Function (functions/mask/matching.py:33-334).

    ``apply`` takes the reference's positional arguments, applies its defaults
    and validation, and runs the step as a C++ autograd node of the extension
    (``mask_loss.mask_matching_autograd``): the forward launches the fused cost
    -> assignment -> loss kernels (and, when the mask logits need a gradient,
    the gradient buffer's zero fill); the node's backward writes the matched
    rows into that buffer and the class-logit gradient.  Returns
    (pred_to_gt, pred_round, layer mask mean, layer dice mean, layer class mean).
    """

    @staticmethod
    def apply(
        mask_logits,  # (L,B,Q,H,W)
        mask_targets,  # (B,H_t,W_t)
        cls_logits,  # (L,B,Q,C)
        cls_targets,  # (B,GT)
        smooth,
        sigmoid_scale,
        dice_scale,
        cls_scale,
        background_index,
        uncertainty_gamma,
        uncertainty_gamma_min,
        normalize_uncertainty,
        inf_thresh,
        num_masks,
        force_unmatched_class_to_background,
        force_unmatched_masks_to_empty,
        K,
        assignment_strategy,
        mask_focal_gamma,
        mask_focal_alpha,
        cls_focal_gamma,
        cls_focal_alpha,
        void_class_index=None,
        label_loss: str = "sigmoid",
    ):
        L, B, Q, h, w = mask_logits.shape
        B_t, H_t, W_t = mask_targets.shape
        assert B == B_t, "Batch size mismatch between logits and targets"

        smooth_val = float(smooth if smooth is not None else 1.0)
        sigmoid_scale_val = float(sigmoid_scale if sigmoid_scale is not None else 1.0)
        dice_scale_val = float(dice_scale if dice_scale is not None else 1.0)
        cls_scale_val = float(cls_scale if cls_scale is not None else 1.0)
        bg = int(background_index if background_index is not None else -1)
        ug, ugm = uncertainty(uncertainty_gamma, uncertainty_gamma_min)
        normalize = bool(normalize_uncertainty if normalize_uncertainty is not None else True)
        inf_thresh_val = float(inf_thresh if inf_thresh is not None else 1e30)
        num_masks_val = float(num_masks if num_masks is not None else -1.0)
        force_cls = bool(force_unmatched_class_to_background
                         if force_unmatched_class_to_background is not None else False)
        force_masks = bool(force_unmatched_masks_to_empty
                           if force_unmatched_masks_to_empty is not None else False)
        strategy = assignment_strategy if assignment_strategy is not None else "global"
        if strategy not in STRATEGIES:
            raise ValueError(f"Unknown assignment_strategy '{strategy}'."
                             f" Expected one of {sorted(STRATEGIES.keys())}")
        K_val = int(K if K is not None else 1)
        if K_val < 0:
            raise ValueError("K must be non-negative")
        mg, ma, cg, ca = focal(mask_focal_gamma, mask_focal_alpha, cls_focal_gamma, cls_focal_alpha)
        C = cls_logits.shape[-1]
        if void_class_index is None:
            void = -1
        else:
            void = int(void_class_index)
            if not (0 <= void < C):
                raise ValueError("incorrect void index")
        use_softmax = label_kind(label_loss)
        if use_softmax and force_cls and void == -1:
            raise ValueError("void_class_index must be provided when using softmax label loss "
                             "and forcing unmatched predictions to background")
        # The void-class check (reference: a synchronous torch.any before any
        # work) runs in the forward's first kernels; the call returns once
        # they are done, with the rest of the forward still queued, and raises
        # ValueError("cls_targets must not contain the void class index").
        return tuple(mask_loss.mask_matching_autograd(
            mask_logits, mask_targets, cls_logits, cls_targets, smooth_val, sigmoid_scale_val,
            dice_scale_val, cls_scale_val, bg, ug, ugm, inf_thresh_val, num_masks_val, force_cls,
            force_masks, K_val, STRATEGIES[strategy], mg, ma, cg, ca, void, use_softmax, normalize,
            void != -1))
