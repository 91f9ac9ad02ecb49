"""MaskMatchingFunction -- reference functions/mask/matching.py:21-334.

Same positional signature, defaults and validation as the reference.  The
differences are on the device side only:

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
  gradient tensor and zero-fills it on a side stream while the assignment
  runs; the first backward then writes only the matched rows into it.
"""
from __future__ import annotations

import torch
from torch.autograd import Function

import mask_loss_amd  # noqa: F401  (registers the `mask_loss` module)
import mask_loss

from .._args import STRATEGIES, focal, label_kind, uncertainty


class MaskMatchingFunction(Function):
    @staticmethod
    def forward(
        ctx,
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
        mask_logits = mask_logits.contiguous()
        mask_targets = mask_targets.contiguous()
        cls_logits = cls_logits.contiguous()
        cls_targets = cls_targets.contiguous()

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

        args = (smooth_val, sigmoid_scale_val, dice_scale_val, cls_scale_val, bg, ug, ugm)
        prefill = None
        if ctx.needs_input_grad[0] and not force_masks:
            prefill = torch.empty_like(mask_logits, memory_format=torch.contiguous_format)
        # The void-class check (reference: a synchronous torch.any before any
        # work) runs in the forward's first kernels; the call returns once
        # they are done, with the rest of the forward still queued, so the
        # host never drains the GPU before launching it.
        check = void != -1
        outs = mask_loss.mask_matching_fused(
            mask_logits, mask_targets, cls_logits, cls_targets, *args, inf_thresh_val,
            num_masks_val, force_cls, force_masks, K_val, STRATEGIES[strategy], mg, ma, cg, ca,
            void, use_softmax, normalize, prefill, check)
        pred_to_gt, pred_round, m, d, c, saved = outs[:6]
        ctx.save_for_backward(mask_logits.detach(), mask_targets.detach(), cls_logits.detach(),
                              cls_targets.detach(), pred_to_gt.detach(), saved)
        # the zero-filled gradient buffer serves the first backward only (a
        # second backward through a retained graph gets a fresh tensor)
        ctx.prefill = prefill
        ctx.bwd_args = (smooth_val, sigmoid_scale_val, dice_scale_val, cls_scale_val, bg, ug, ugm,
                        num_masks_val, force_cls, force_masks, mg, ma, cg, ca, void, use_softmax,
                        normalize)
        if check and int(outs[6][0]) == 1:
            raise ValueError("cls_targets must not contain the void class index")
        ctx.mark_non_differentiable(pred_to_gt, pred_round)
        # no zero gradients for the integer outputs (or unused means)
        ctx.set_materialize_grads(False)
        return pred_to_gt, pred_round, m, d, c

    @staticmethod
    def backward(ctx, _, __, grad_layer_mask_mean, grad_layer_dice_mean, grad_layer_cls_mean):
        mask_logits, mask_targets, cls_logits, cls_targets, pred_to_gt, saved = ctx.saved_tensors
        prefill, ctx.prefill = ctx.prefill, None

        def g(x):
            return x.detach().float().contiguous() if x is not None else \
                torch.zeros(mask_logits.shape[0], device=mask_logits.device)

        grad_mask, grad_cls = mask_loss.mask_matching_backward_fused(
            g(grad_layer_mask_mean), g(grad_layer_dice_mean), g(grad_layer_cls_mean),
            mask_logits, mask_targets, cls_logits, cls_targets, pred_to_gt, *ctx.bwd_args, saved,
            prefill)
        return (grad_mask, None, grad_cls) + (None,) * 21
